"""The fused decode attention on the GPU against the oracle's portable chain
(llama.py's decode attention: RoPE, blended cache write, GQA sdpa), across
head groupings 1/2/4/8, cache lengths that do and do not fill the last
chunk, batches with per-sequence positions, fractional write masks,
per-head attention masks, float32/float16/bfloat16, every pass count, and
functional as well as donated (in-place) caches.  The attention output is
within the dtype's tolerance; the updated float16/bfloat16 caches are
bit-identical (float32 ones to the last ulps)."""

from __future__ import annotations

import numpy as np
import pytest

import attention_cases
from chomikgrad import realize
from chomikgrad.dtypes import BFLOAT16, bf16_to_float32

pytestmark = pytest.mark.gpu


def as_float(values):
    values = np.asarray(values)
    return bf16_to_float32(values) if values.dtype == BFLOAT16 else values.astype(np.float32)


@pytest.mark.parametrize("passes", [0, 1, 4, -2, "stream8", "stream768", "stream8-u4"])
@pytest.mark.parametrize("case", attention_cases.CASES, ids=lambda c: c.name)
def test_decode_attention_matches_oracle(hip, case, passes, monkeypatch):
    """passes: the chunk kernel's passes per workgroup (0 = chosen), -2 the
    MFMA kernel where it applies (16-bit caches of at most 768 rows), or the
    streaming kernel aiming at 8 workgroups (one or two ranges per KV head,
    many tiles) or 768 (many short ranges, combined), with two passes per
    tile or, for "-u4", four."""
    from chomikgrad import _planner

    print(f"[gpu case] decode attention {case.name} passes={passes}", flush=True)
    if isinstance(passes, str):
        wgs, _, unroll = passes[len("stream"):].partition("-u")
        monkeypatch.setattr(_planner, "DECODE_ATTN_PASSES", -1)
        monkeypatch.setattr(_planner, "DECODE_ATTN_STREAM_WGS", int(wgs))
        monkeypatch.setattr(_planner, "DECODE_ATTN_STREAM_UNROLL", int(unroll or 2))
    else:
        monkeypatch.setattr(_planner, "DECODE_ATTN_PASSES", passes)
    outputs, dynamic, caches = attention_cases.build(case)
    expected = realize(*outputs, compiler="cpu")
    tolerance = attention_cases.tolerance(case)
    for donate in (False, True):
        program = hip.compile([o._node for o in outputs], [t._node for t in dynamic],
                              donate=[t._node for t in caches] if donate else ())
        assert "decode_attention" in program.source
        bound = {t._node: hip.device.array(t._node.numpy_value()) for t in dynamic}
        native = program.run(bound, synchronize=True)
        got = [hip.device.to_numpy(value) for value in native]
        np.testing.assert_allclose(as_float(got[0]), as_float(expected[0]), **tolerance)
        for value, reference in zip(got[1:], expected[1:]):
            if value.dtype == np.float32:
                # the oracle's float32 RoPE is a BLAS matmul whose FMA use
                # depends on the host CPU: agree to the last ulps only
                np.testing.assert_allclose(value, reference, rtol=1e-6, atol=1e-7)
            else:  # products of half-precision values are exact in float32
                np.testing.assert_array_equal(value.view(np.uint8), np.asarray(reference).view(np.uint8))
        if donate:  # the returned caches are the bound input buffers
            assert native[1] is bound[caches[0]._node] and native[2] is bound[caches[1]._node]
        # a second run on the updated caches (tickets reset, partials reused)
        again = [hip.device.to_numpy(v) for v in program.run(bound, synchronize=True)]
        if not donate:
            np.testing.assert_array_equal(again[0].view(np.uint8), got[0].view(np.uint8))
