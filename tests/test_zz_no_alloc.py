"""chip_greedy_advance_noalloc against chip_greedy_advance, through the C ABI.

The allocation-free variant keeps the kernel's per-row key words and
tickets in a static device array instead of scratch the library allocates.
Both entry points run the same kernel on copies of the same inputs and must
leave bit-identical tokens, history, positions and masks; the tokens must
also be NumPy's argmax (first maximum, a NaN counting as the maximum).  Two
calls in a row, the second smaller (fewer rows, fewer columns, other dtypes),
show that the shared static array is left clean between calls; a request
above its 1024-row limit is refused before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from chomikgrad.dtypes import BFLOAT16, bf16_to_float32, dtype_code, to_bf16

pytestmark = pytest.mark.gpu


def _case(rows, cols, logits_dtype, mask_dtype, cache, step, seed):
    rng = np.random.default_rng(seed)
    logits = rng.normal(size=(rows, cols)).astype(np.float32)
    logits[0, [7, cols - 3]] = 9.0           # a tie: the first index wins
    if rows > 2:
        logits[2, [11, 40]] = np.nan         # a NaN is the maximum, the first NaN wins
    host = {
        "logits": to_bf16(logits) if logits_dtype == BFLOAT16 else logits.astype(logits_dtype),
        "tokens": np.full(rows, -1, np.int32),
        "history": np.full((step + 2) * rows, -1, np.int32),
        "position": rng.integers(0, cache - 2, rows).astype(np.int32),
    }
    attention = np.where(np.arange(cache)[None, :] <= host["position"][:, None], 0.0, -1e4).astype(np.float32)
    write = (np.arange(cache)[None, :] == host["position"][:, None]).astype(np.float32)
    cast = (lambda v: to_bf16(v)) if mask_dtype == BFLOAT16 else (lambda v: v.astype(mask_dtype))
    host["attention"] = cast(attention.reshape(rows, 1, 1, cache))
    host["write"] = cast(write.reshape(rows, 1, cache, 1))
    return host


def _run(hip, entry, host, step, cache, mask_dtype):
    device = {name: hip.device.array(value) for name, value in host.items()}
    rows, cols = host["logits"].shape
    hip.lib.call(entry, ctypes.c_void_p(device["logits"].ptr), dtype_code(host["logits"].dtype),
                 ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_void_p(device["tokens"].ptr),
                 ctypes.c_void_p(device["history"].ptr), ctypes.c_int64(step),
                 ctypes.c_void_p(device["position"].ptr), ctypes.c_void_p(device["attention"].ptr),
                 ctypes.c_int64(cache), ctypes.c_void_p(device["write"].ptr), ctypes.c_int64(cache),
                 dtype_code(np.dtype(mask_dtype)), ctypes.c_int64(cache))
    hip.device.synchronize()
    return {name: hip.device.to_numpy(array) for name, array in device.items()}


def _expected_tokens(logits):
    values = bf16_to_float32(logits) if logits.dtype == BFLOAT16 else logits.astype(np.float32)
    return np.argmax(values, axis=1)  # NumPy: first maximum, a NaN counts as the maximum


@pytest.mark.parametrize("call", [0, 1])
def test_noalloc_greedy_advance_matches_allocating_entry(hip, call):
    # call 0: 8 rows x 32000 float16 logits, float16 masks; call 1 (run
    # right after it, on the same static array): 3 rows x 1000 bfloat16
    # logits, float32 masks.
    rows, cols, ldt, mdt, cache, step = [(8, 32000, np.float16, np.float16, 64, 3),
                                         (3, 1000, BFLOAT16, np.float32, 40, 0)][call]
    print(f"[gpu case] no-alloc greedy advance call {call}: {rows} x {cols}", flush=True)
    host = _case(rows, cols, ldt, mdt, cache, step, seed=call)
    plain = _run(hip, "chip_greedy_advance", host, step, cache, mdt)
    static = _run(hip, "chip_greedy_advance_noalloc", host, step, cache, mdt)
    for name in host:  # bit for bit (the logits hold NaNs, so compare bytes)
        got, want = np.ascontiguousarray(static[name]), np.ascontiguousarray(plain[name])
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), name
    expected = _expected_tokens(host["logits"])
    assert np.array_equal(static["tokens"], expected)
    assert np.array_equal(static["history"][step * rows:(step + 1) * rows], expected)
    assert np.array_equal(static["position"], host["position"] + 1)
    new = host["position"] + 1
    attention = static["attention"].reshape(rows, cache)
    write = static["write"].reshape(rows, cache)
    if write.dtype == BFLOAT16:
        attention, write = bf16_to_float32(attention), bf16_to_float32(write)
    for r in range(rows):
        assert attention[r, new[r]] == 0 and write[r, new[r]] == 1 and write[r, new[r] - 1] == 0


def test_noalloc_rejects_rows_beyond_static_scratch(hip):
    print("[gpu case] no-alloc greedy advance: 1025 rows refused", flush=True)
    # Real buffers pass the argument checks; the row count is refused before
    # any launch, so their sizes never matter.
    logits = hip.device.array(np.zeros(16, np.float16))
    tokens = hip.device.array(np.zeros(16, np.int32))
    null = ctypes.c_void_p(None)
    with pytest.raises(RuntimeError, match="1024"):
        hip.lib.call("chip_greedy_advance_noalloc", ctypes.c_void_p(logits.ptr), dtype_code(np.dtype(np.float16)),
                     ctypes.c_int64(1025), ctypes.c_int64(16), ctypes.c_void_p(tokens.ptr), null,
                     ctypes.c_int64(0), null, null, ctypes.c_int64(0), null, ctypes.c_int64(0),
                     dtype_code(np.dtype(np.float16)), ctypes.c_int64(0))
    hip.device.synchronize()
