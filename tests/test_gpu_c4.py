"""C4 (Llama-3.2-1B shape, bfloat16, batch 8 over 4096-position caches, tied
embedding/LM head, RoPE theta 5e5) on the hip plugin:

* every per-layer shape at its full size, two layers deep, against the
  oracle: logits within the bf16 tolerance and no less accurate than the
  oracle against float32; cache rows not written bit-identical, written
  rows within one ulp (layer 0) or the tolerance (later layers);
* the full 16-layer model, batched, and one sequence of it decoded alone:
  each at least as close to the same step evaluated in float32 as the
  oracle's bfloat16 evaluation is."""

from __future__ import annotations

import numpy as np
import pytest

import c4_case
from chomikgrad import Tensor, realize
from chomikgrad.dtypes import bf16_to_float32
from chomikgrad.llama import LlamaDecoderStep

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2  # the north-star float16/bfloat16 logit tolerance


def test_c4_shapes_match_oracle(hip):
    """The oracle rounds every intermediate of the softmax chain to bfloat16;
    the fused decode attention keeps it in float32.  So the GPU is checked
    against the oracle at the north-star tolerance for all but a sliver of
    the million logits, and against the same inputs evaluated in float32:
    the GPU's error there must not exceed the bfloat16 oracle's own."""
    print("[gpu case] C4 shapes (2 layers) vs oracle", flush=True)
    cfg, _, leaves, caches, outputs = c4_case.build(layers=2)
    expected = realize(*outputs, compiler="cpu")
    program_out = realize(*outputs, compiler="hip")
    got_logits, want_logits = bf16_to_float32(program_out[0]), bf16_to_float32(expected[0])
    outside = np.abs(got_logits - want_logits) > ATOL + RTOL * np.abs(want_logits)
    assert outside.mean() < 0.01, f"{outside.mean():.4f} of the logits outside the tolerance"
    np.testing.assert_allclose(got_logits, want_logits, atol=4 * ATOL, rtol=RTOL)
    margin = np.sort(want_logits, axis=-1)[:, -1] - np.sort(want_logits, axis=-1)[:, -2]
    clear = margin > 0.05
    assert np.array_equal(got_logits.argmax(-1)[clear], want_logits.argmax(-1)[clear])
    # Cache rows not written this step are bit-identical.  The written row
    # is the layer's k/v projection: in layer 0 (same input on both sides;
    # only the float32 sum order differs from NumPy's) within one bfloat16
    # ulp, in later layers (inputs already within tolerance) within the logit
    # tolerance.
    positions = np.asarray(leaves[4]._node.numpy_value())
    for index, (value, reference) in enumerate(zip(program_out[1:], expected[1:])):
        value, reference = np.asarray(value), np.asarray(reference)
        bound = dict(rtol=2 ** -7, atol=0) if index < 2 else dict(rtol=RTOL, atol=ATOL)
        for b, p in enumerate(positions):
            keep = np.ones(c4_case.CONTEXT, bool)
            keep[p] = False
            np.testing.assert_array_equal(value[b][:, keep].view(np.uint16), reference[b][:, keep].view(np.uint16))
            np.testing.assert_allclose(bf16_to_float32(value[b][:, p]), bf16_to_float32(reference[b][:, p]), **bound)
    # the same inputs in float32: the GPU is at least as close as the oracle
    truth = np.asarray(realize(c4_case.build(layers=2, float32=True)[4][0], compiler="cpu")[0])
    gpu_error = np.abs(got_logits - truth).mean()
    oracle_error = np.abs(want_logits - truth).mean()
    print(f"mean |logit error| vs float32: hip {gpu_error:.5f}, bf16 oracle {oracle_error:.5f}", flush=True)
    # The tolerance measured against float32 itself: the bfloat16 oracle misses
    # it for a comparable share of logits, so no bfloat16 evaluation can be
    # held to it on every logit.
    def share_outside(values):
        return float((np.abs(values - truth) > ATOL + RTOL * np.abs(truth)).mean())
    print(f"share outside atol {ATOL}/rtol {RTOL}: hip vs oracle {outside.mean():.5f}, "
          f"hip vs float32 {share_outside(got_logits):.5f}, oracle vs float32 {share_outside(want_logits):.5f}; "
          f"max |hip - oracle| {np.abs(got_logits - want_logits).max():.4f}", flush=True)
    assert gpu_error <= oracle_error * 1.05


def test_c4_full_model_batch_equals_single_sequences(hip):
    """The full 16-layer model, batch 8.  Sixteen layers of bfloat16 rounding
    put any bfloat16 evaluation ~0.02 (mean |logit error|) away from the same
    step in float32, so sequence 0 is checked against that float32 step: the
    batched run and a batch-1 run of the same sequence on the GPU must each
    be at least as close to it as the oracle's bfloat16 evaluation (the
    reference's algorithm) is, and pick the same token where float32's top two
    logits are clearly apart."""
    from chomikgrad.dtypes import bf16_to_float32 as widen

    print("[gpu case] C4 full model: batched and batch-1 steps vs float32 and the oracle", flush=True)
    cfg, weights, leaves, caches, outputs = c4_case.build(layers=16)
    batched = bf16_to_float32(realize(*outputs[:1], compiler="hip")[0])
    host = [np.asarray(t._node.numpy_value()) for t in leaves]
    cache_host = [np.asarray(c._node.numpy_value()) for c in caches]

    def sequence0(step_weights, dtype, compiler, cast=lambda a: a):
        small = [Tensor(cast(v[:1]) if i in (1, 2, 3) else v[:1], copy=False) for i, v in enumerate(host[:4])]
        small.append(Tensor(np.asarray(host[4][0], np.int32), copy=False))
        own = [Tensor(cast(c[:1]), copy=False) for c in cache_host]
        step = LlamaDecoderStep(cfg, step_weights, cache_length=c4_case.CONTEXT, dtype=dtype)
        out = step(*small[:4], list(zip(own[::2], own[1::2])), position=small[4])
        return np.asarray(realize(out[0], compiler=compiler)[0])

    alone = bf16_to_float32(sequence0(weights, cache_host[0].dtype, "hip"))[0]
    oracle = bf16_to_float32(sequence0(weights, cache_host[0].dtype, "cpu"))[0]
    wide = {name: Tensor(widen(np.asarray(t._node.numpy_value())), copy=False) for name, t in weights.items()}
    wide["lm_head.weight"] = wide["model.embed_tokens.weight"]
    truth = sequence0(wide, np.float32, "cpu", cast=widen)[0]
    reference_error = np.abs(oracle - truth).mean()
    for name, logits in (("batched", batched[0]), ("batch-1", alone)):
        error = np.abs(logits - truth).mean()
        print(f"{name}: mean |logit error| vs float32 {error:.5f} (bf16 oracle {reference_error:.5f})", flush=True)
        assert error <= 1.1 * reference_error
        top = np.sort(truth)[-2:]
        if top[1] - top[0] > 0.1:
            assert logits.argmax() == truth.argmax()
