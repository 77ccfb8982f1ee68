"""The hip plugin against the oracle on the six IR ops and the fused kernels
(plugin conformance, after the reference's tests/test_cuda.py and
tests/test_mlx.py, aimed at compiler="hip")."""

from __future__ import annotations

import numpy as np
import pytest

from chomikgrad import Tensor, compile_graph, realize
from chomikgrad.dtypes import BFLOAT16, as_dtype, bf16_to_float32, dtype_name, to_bf16
from chomikgrad.hip_backend import HIPArray

pytestmark = pytest.mark.gpu


def announce(name):
    print(f"[gpu case] {name}", flush=True)


def as_float(values):
    values = np.asarray(values)
    return bf16_to_float32(values) if values.dtype == BFLOAT16 else values.astype(np.float32)


def both(*tensors):
    return realize(*tensors, compiler="hip"), realize(*tensors, compiler="cpu")


def test_six_ir_operations_and_gather_match_cpu(hip):
    announce("six ops + gather")
    left = Tensor([[1.0, -2.0, 0.5], [3.0, 4.0, -1.0]], dtype=np.float32)
    right = Tensor([[2.0, 1.0], [-1.0, 0.5], [3.0, -2.0]], dtype=np.float32)
    result = ((left @ right).relu() + 0.25).permute(1, 0).reshape(1, 4).sum(axis=1)
    program = compile_graph(result, compiler="hip")
    np.testing.assert_allclose(program()[0], result.numpy(compiler="cpu"), rtol=1e-5, atol=1e-6)
    assert "fused_elementwise" in program.source and "matmul" in program.source
    table = Tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dtype=np.float32)
    gathered = table.gather(Tensor(np.array([[2, 0, -3]], dtype=np.int32), copy=False))
    gather_program = compile_graph(gathered, compiler="hip")
    assert "gather" in gather_program.source
    np.testing.assert_allclose(gather_program()[0], [[[5.0, 6.0], [1.0, 2.0], [1.0, 2.0]]])


def test_gather_index_outside_table_raises_index_error(hip):
    announce("gather out of range -> IndexError")
    table = Tensor(np.arange(6, dtype=np.float32).reshape(3, 2))
    with pytest.raises(IndexError):
        table.gather(Tensor(np.array([5], dtype=np.int64))).numpy(compiler="hip")
    # the error is cleared: the next program runs normally
    np.testing.assert_allclose(table.gather(Tensor(np.array([1], np.int64))).numpy(compiler="hip"), [[2.0, 3.0]])


@pytest.mark.parametrize("dtype", [np.float32, np.float16, BFLOAT16])
def test_batched_matmul_matches_cpu(hip, dtype):
    announce(f"batched matmul {np.dtype(dtype)}")
    rng = np.random.default_rng(19)
    left = Tensor(rng.normal(size=(2, 4, 3, 5)).astype(np.float32), dtype=dtype)
    right = Tensor(rng.normal(size=(2, 4, 5, 6)).astype(np.float32), dtype=dtype)
    weight = Tensor(rng.normal(size=(5, 7)).astype(np.float32), dtype=dtype)
    outputs = [left @ right, left @ weight, Tensor(rng.normal(size=(1, 3, 5)).astype(np.float32), dtype=dtype) @ weight]
    got, expected = both(*outputs)
    tolerance = 1e-5 if dtype == np.float32 else 1e-2
    for g, e in zip(got, expected):
        np.testing.assert_allclose(as_float(g), as_float(e), rtol=tolerance, atol=tolerance)


def test_dynamic_input_and_deferred_synchronization(hip):
    announce("dynamic input rebinding")
    source = Tensor([1.0, 2.0], dtype=np.float32)
    program = compile_graph(source * 2.0, compiler="hip", dynamic_inputs=(source,))
    replacement = hip.device.array(np.array([3.0, 4.0], dtype=np.float32))
    native = program.run({source._node: replacement}, synchronize=False)[0]
    program.device.synchronize()
    assert isinstance(native, HIPArray)
    np.testing.assert_allclose(program.device.to_numpy(native), [6.0, 8.0])
    np.testing.assert_allclose(program()[0], [2.0, 4.0])
    assert program.inputs == (source._node,)
    assert program.device.argmax(native) == 1
    np.testing.assert_array_equal(program.device.argmax_last_axis(native), 1)


def test_argmax_follows_numpy_first_occurrence_and_nan(hip):
    announce("argmax ties and NaN")
    device = hip.device
    values = np.array([[1.0, 5.0, 5.0, 2.0], [np.nan, 1.0, np.nan, 9.0], [-np.inf] * 4], dtype=np.float32)
    native = device.array(values)
    np.testing.assert_array_equal(device.argmax_last_axis(native), values.argmax(axis=-1))
    big = np.random.default_rng(0).normal(size=32000).astype(np.float16)
    big[[7, 31000]] = np.float16(60000.0)
    assert device.argmax(device.array(big)) == 7


def test_copy_false_observes_host_mutation(hip):
    announce("copy=False re-uploads")
    source = np.array([1.0, 2.0], dtype=np.float32)
    tensor = Tensor(source, copy=False)
    np.testing.assert_allclose(tensor.numpy(compiler="hip"), [1.0, 2.0])
    source[0] = 9.0
    np.testing.assert_allclose((tensor * 1.0).numpy(compiler="hip"), [9.0, 2.0])


def test_softmax_reductions_and_elementwise_chains(hip):
    announce("softmax/reduce/elementwise")
    rng = np.random.default_rng(29)
    for dtype in (np.float32, np.float16):
        source = Tensor(rng.normal(size=(3, 5, 64)).astype(dtype))
        outputs = [source.softmax(axis=-1), source.softmax(axis=1), source.max(axis=(0, 2), keepdims=True),
                   source.sum(), (source.exp() * 2.0 - source.relu().sqrt()).mean(axis=-1),
                   source.log_softmax(axis=-1), source.layer_norm(Tensor(np.ones(64, dtype)), Tensor(np.zeros(64, dtype)))]
        got, expected = both(*outputs)
        tolerance = 2e-5 if dtype == np.float32 else 2e-3
        for g, e in zip(got, expected):
            np.testing.assert_allclose(as_float(g), as_float(e), rtol=tolerance, atol=tolerance)


def test_structural_program_cache_and_leaf_aliasing(hip):
    announce("program cache")
    first = Tensor([1.0, 2.0], dtype=np.float32).relu().softmax()
    first.numpy(compiler="hip")
    size = hip.cache_size
    Tensor([3.0, 4.0], dtype=np.float32).relu().softmax().numpy(compiler="hip")
    assert hip.cache_size == size
    left, right = Tensor([1.0, 2.0], dtype=np.float32), Tensor([10.0, 20.0], dtype=np.float32)
    np.testing.assert_allclose((left + left).numpy(compiler="hip"), [2.0, 4.0])
    np.testing.assert_allclose((left + right).numpy(compiler="hip"), [11.0, 22.0])


def test_programs_sharing_a_plan_and_repeated_runs(hip):
    """Programs of one structure share a plan (the structural program
    cache): running one after the other rebinds each program's own leaves,
    and a run repeated with the same device arrays (the resident-loop fast
    path) reads what was uploaded into them since."""
    announce("shared plans and repeated runs")
    a = Tensor(np.array([1.0, 2.0], np.float32))
    b = Tensor(np.array([10.0, 20.0], np.float32))
    pa = compile_graph((a * 2.0).relu(), compiler="hip")
    pb = compile_graph((b * 2.0).relu(), compiler="hip")
    for _ in range(2):
        np.testing.assert_allclose(pa()[0], [2.0, 4.0])
        np.testing.assert_allclose(pb()[0], [20.0, 40.0])
    source = Tensor(np.array([1.0, -3.0], np.float32))
    program = compile_graph((source * 3.0).relu(), compiler="hip", dynamic_inputs=(source,))
    bound = hip.device.array(np.array([1.0, 2.0], np.float32))
    out = [hip.device.empty((2,), np.float32)]
    first = program.run({source._node: bound}, out=out, synchronize=True)
    np.testing.assert_allclose(hip.device.to_numpy(first[0]), [3.0, 6.0])
    hip.device.upload(bound, np.array([-1.0, 5.0], np.float32))
    again = program.run({source._node: bound}, out=out, synchronize=True)
    assert again[0] is first[0]
    np.testing.assert_allclose(hip.device.to_numpy(again[0]), [0.0, 15.0])
    other = hip.device.array(np.array([4.0, 4.0], np.float32))
    np.testing.assert_allclose(hip.device.to_numpy(program.run({source._node: other}, out=out, synchronize=True)[0]),
                               [12.0, 12.0])
    np.testing.assert_allclose(hip.device.to_numpy(program.run({source._node: bound}, out=out, synchronize=True)[0]),
                               [0.0, 15.0])


@pytest.mark.parametrize("dtype", [np.float32, np.float16, BFLOAT16])
@pytest.mark.parametrize("rows,layout", [(1, "sequence")] + [(r, l) for r in (2, 3, 5, 8)
                                                            for l in ("sequence", "batch", "batch-row-exact")])
def test_gemv_linear_variants(hip, dtype, rows, layout, monkeypatch):
    """Few-row linears with RMSNorm prologue, residual and SiLU-pair
    epilogues against the oracle.  ``sequence``: x of shape (1, rows, K), the
    positions of one sequence (the row-exact kernel for 16-bit types);
    ``batch``: (rows, 1, K), independent sequences on the MFMA kernel;
    ``batch-row-exact``: the same on the row-exact kernel, which the planner
    picks for narrow batch matrices.  One row is the same graph in every
    layout."""
    from chomikgrad import _planner

    monkeypatch.setattr(_planner, "GEMV_BATCH_ROW_EXACT", layout == "batch-row-exact")
    monkeypatch.setattr(hip, "_program_cache", {})  # plans depend on the setting, the cache key does not
    announce(f"gemv {np.dtype(dtype)} rows={rows} {layout}")
    rng = np.random.default_rng(rows)
    K, N = 512, 384
    shape = (1, rows) if layout == "sequence" else (rows, 1)
    x = Tensor(rng.normal(size=shape + (K,)).astype(np.float32), dtype=dtype)
    h = Tensor(rng.normal(size=shape + (N,)).astype(np.float32), dtype=dtype)
    norm = Tensor(np.ones(K, np.float32), dtype=dtype)
    w1 = Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype)
    w2 = Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype)
    w3 = Tensor((rng.normal(size=(K, N)) * 0.05).astype(np.float32), dtype=dtype)
    variance = (x * x).mean(axis=-1, keepdims=True)
    normed = x / (variance + 1e-5).sqrt() * norm
    normed._node.lowering = ("rms_norm", (x._node, norm._node), 1e-5)
    gate = normed @ w1.T
    act = gate / (1 + (-gate).exp()) * (normed @ w2.T)
    outputs = [x @ w1.T, h + (x @ w1.T), act, act @ w3.T]
    program = compile_graph(*outputs, compiler="hip")
    assert "gemv" in program.source
    if dtype != np.float32 and rows > 1:
        assert ("row_exact" in program.source) == (layout != "batch")
    got = program()
    expected = realize(*outputs, compiler="cpu")
    tolerance = 1e-4 if dtype == np.float32 else 3e-2
    for g, e in zip(got, expected):
        np.testing.assert_allclose(as_float(g), as_float(e), rtol=tolerance, atol=tolerance)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("rows", [2, 8])
@pytest.mark.parametrize("K,N", [(8192, 384), (4096, 256)], ids=["k8192", "k4096"])
def test_gemv_split_over_blocks(hip, dtype, rows, K, N):
    """MFMA GEMVs whose column tiles are shared by several blocks (each over
    a share of K, the last block to finish adds the partials in block order):
    plain, residual and SiLU-pair epilogues and a narrower GEMV sharing the
    workspace, against the oracle; a second run (tickets reset) is
    bit-identical."""
    from chomikgrad import _planner

    announce(f"gemv split {np.dtype(dtype)} rows={rows} K={K} N={N}")
    rng = np.random.default_rng(K + rows)
    x = Tensor(rng.normal(size=(rows, 1, K)).astype(np.float32), dtype=dtype)  # a batch of sequences
    h = Tensor(rng.normal(size=(rows, 1, N)).astype(np.float32), dtype=dtype)
    w1 = Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype)
    w2 = Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype)
    # a GEMV of another width on its own input shares the workspace
    z = Tensor(rng.normal(size=(rows, 1, K)).astype(np.float32), dtype=dtype)
    w3 = Tensor((rng.normal(size=(160, K)) * 0.05).astype(np.float32), dtype=dtype)
    gate = x @ w1.T
    outputs = [x @ w2.T, h + (x @ w1.T), gate / (1 + (-gate).exp()) * (x @ w2.T), z @ w3.T]
    program = compile_graph(*outputs, compiler="hip")
    gemvs = [s for s in program._planned.steps if s.kind == _planner.K_GEMV]
    assert gemvs and all(s.attrs.get("blocks", 1) > 1 for s in gemvs)
    got = program()
    expected = realize(*outputs, compiler="cpu")
    for g, e in zip(got, expected):
        np.testing.assert_allclose(as_float(g), as_float(e), rtol=3e-2, atol=3e-2)
    again = program()
    for g, a in zip(got, again):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint8), np.asarray(a).view(np.uint8))


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("K", [320, 768, 2048])
def test_row_gemv_rmsnorm_prologue_equals_separate_norm(hip, dtype, K, monkeypatch):
    """One decode row: the RMSNorm folded into the row GEMV's prologue gives
    the bits of the separate rms_norm step followed by the same GEMV.  The
    prologue takes the mean of a power-of-two K by scaling (K = 2048, the
    C2 width) and divides otherwise (K = 320 and 768, whose rows also end
    inside a 16-byte vector group), and its quotient routine runs on the
    hardware reciprocal of rn.  Inputs are multiples of 1/8 in [-2, 2], so
    every float32 sum of squares is exact in any order and both paths round
    the same total; the norm weight is not constant."""
    from chomikgrad import _planner

    monkeypatch.setattr(hip, "_program_cache", {})
    announce(f"gemv row prologue {np.dtype(dtype)} K={K}")
    rng = np.random.default_rng(K)
    N = 200
    x = Tensor((rng.integers(-16, 17, size=(1, 1, K)) / 8).astype(np.float32), dtype=dtype)
    h = Tensor(rng.normal(size=(1, 1, N)).astype(np.float32), dtype=dtype)
    norm = Tensor(rng.normal(1.0, 0.3, size=K).astype(np.float32), dtype=dtype)
    w1, w2, w3 = (Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype) for _ in range(3))
    variance = (x * x).mean(axis=-1, keepdims=True)
    normed = x / (variance + 1e-5).sqrt() * norm
    normed._node.lowering = ("rms_norm", (x._node, norm._node), 1e-5)
    gate = normed @ w1.T
    outputs = [h + normed @ w3.T, gate / (1 + (-gate).exp()) * (normed @ w2.T)]
    fused = compile_graph(*outputs, compiler="hip")
    assert " rms_norm(" not in fused.source and fused.source.count("gemv[rms_norm") == 2
    assert "row_exact" not in fused.source
    got = fused()
    monkeypatch.setattr(_planner, "fuse_rmsnorm_prologue", lambda steps, outputs: steps)
    monkeypatch.setattr(hip, "_program_cache", {})  # plan again rather than reuse the fused program
    separate = compile_graph(*outputs, compiler="hip")
    assert " rms_norm(" in separate.source
    want = separate()
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint16), np.asarray(w).view(np.uint16))
    expected = realize(*outputs, compiler="cpu")
    for g, e in zip(got, expected):
        np.testing.assert_allclose(as_float(g), as_float(e), rtol=3e-2, atol=3e-2)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("rows,K", [(2, 96), (3, 128), (5, 256), (8, 512), (8, 1024)])
def test_mfma_gemv_rmsnorm_prologue_equals_separate_norm(hip, dtype, rows, K, monkeypatch):
    """A batch's RMSNorm folded into the MFMA GEMV as its prologue gives the
    bits of the separate rms_norm step followed by the same GEMV.  The inputs
    are multiples of 1/8 in [-2, 2], so every square and every float32 sum
    of squares is exact in any order and both paths round the same total;
    the norm weight is not constant, so a misplaced weight or row shows.
    K = 96 ends inside a register chunk; K = 128 and 256 put two and four
    column tiles in a block; K = 1024 splits K over eight waves (both paths
    split K alike at these sizes, so the sums are added in the same order)."""
    from chomikgrad import _planner

    monkeypatch.setattr(_planner, "GEMV_BATCH_ROW_EXACT", False)  # N = 208 would take the row-exact kernel
    monkeypatch.setattr(hip, "_program_cache", {})
    announce(f"gemv mfma prologue {np.dtype(dtype)} rows={rows} K={K}")
    rng = np.random.default_rng(K + rows)
    N = 208  # 13 column tiles: a partial block of tiles where several share a block
    x = Tensor((rng.integers(-16, 17, size=(rows, 1, K)) / 8).astype(np.float32), dtype=dtype)
    h = Tensor(rng.normal(size=(rows, 1, N)).astype(np.float32), dtype=dtype)
    norm = Tensor(rng.normal(1.0, 0.3, size=K).astype(np.float32), dtype=dtype)
    w1, w2, w3 = (Tensor((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype=dtype) for _ in range(3))
    variance = (x * x).mean(axis=-1, keepdims=True)
    normed = x / (variance + 1e-5).sqrt() * norm
    normed._node.lowering = ("rms_norm", (x._node, norm._node), 1e-5)
    gate = normed @ w1.T
    outputs = [h + normed @ w3.T, gate / (1 + (-gate).exp()) * (normed @ w2.T)]
    fused = compile_graph(*outputs, compiler="hip")
    assert " rms_norm(" not in fused.source and fused.source.count("gemv[rms_norm") == 2
    got = fused()
    monkeypatch.setattr(_planner, "fuse_rmsnorm_prologue", lambda steps, outputs: steps)
    monkeypatch.setattr(hip, "_program_cache", {})  # plan again rather than reuse the fused program
    separate = compile_graph(*outputs, compiler="hip")
    assert " rms_norm(" in separate.source
    want = separate()
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint16), np.asarray(w).view(np.uint16))
    expected = realize(*outputs, compiler="cpu")
    for g, e in zip(got, expected):
        np.testing.assert_allclose(as_float(g), as_float(e), rtol=3e-2, atol=3e-2)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("shape", [(37, 200, 72), (130, 96, 512), (9, 4100, 264), (2048, 4096, 256),
                                   (1000, 16384, 320), (2000, 2048, 192)],
                         ids=["ragged", "tall", "wide", "large-tiles", "8-wave-tiles", "8-wave-128-tiles"])
def test_gemm_linear_matches_fp32_reference(hip, dtype, shape):
    """Linears with more than 8 rows run the MFMA GEMM (K_GEMM): fp32
    accumulation of the 16-bit operands and one rounding, against a float32
    matmul of the same rounded inputs.  Shapes cover ragged M/N/K edges, the
    64x64 and 128x128 tiles, the 8-wave 256x128 tiles (512 of those: 4 x
    128, the last row of tiles ragged) and 8-wave 128x128 tiles (256, the
    last row ragged), and K a multiple of 8 but not of the 64-column
    stage."""
    M, N, K = shape
    announce(f"gemm {dtype_name(dtype)} M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    xh = as_dtype(rng.normal(size=(1, M, K)).astype(np.float32), dtype)
    wh = as_dtype((rng.normal(size=(N, K)) * 0.05).astype(np.float32), dtype)
    x, w = Tensor(xh), Tensor(wh)
    program = compile_graph(x @ w.T, compiler="hip")
    assert "gemm" in program.source
    (got,) = program()
    xf = as_float(xh).reshape(M, K)
    wf = as_float(wh)
    expected = xf @ wf.T
    tolerance = 1e-2 if dtype == np.float16 else 2e-2
    np.testing.assert_allclose(as_float(got).reshape(M, N), expected, rtol=tolerance, atol=tolerance)


def _sdpa_graph(q, k, v, mask, heads, dtype):
    """The llama builder's portable GQA attention, tagged ``sdpa``."""
    kv = k.shape[1]
    ones = Tensor(np.ones((1, 1, heads // kv, 1, 1), np.float32), dtype=dtype)

    def repeat(x):
        b, _, t, hd = x.shape
        return (x.reshape(b, kv, 1, t, hd) * ones).reshape(b, heads, t, hd)

    scores = (q @ repeat(k).transpose(-2, -1)) / np.sqrt(64) + mask
    out = scores.softmax(axis=-1) @ repeat(v)
    out._node.lowering = ("sdpa", (q._node, k._node, v._node, mask._node), 1 / np.sqrt(64))
    return out


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("T,mask_kind,H", [(100, "causal", 8), (300, "causal", 8), (70, "dense", 8),
                                           (400, "causal", 16)])
def test_prefill_attention_matches_oracle(hip, dtype, T, mask_kind, H):
    """Prefill attention (K_SDPA with 16+ query rows, head size 64) runs the
    MFMA kernel: a captured causal triangle is proved and applied
    arithmetically (tiles above the diagonal skipped); any other mask is read
    from memory.  Ragged T covers partial query and key tiles; 8 (16) query
    heads over 2 (4) KV heads covers GQA.  16 heads over an even number of
    128-row query tiles take the balanced block order (tile qt beside tile
    Q-1-qt), the others the plain order."""
    announce(f"prefill attention {dtype_name(dtype)} T={T} {mask_kind} H={H}")
    rng = np.random.default_rng(T)
    KV = H // 4
    q = Tensor(as_dtype(rng.normal(size=(1, H, T, 64)).astype(np.float32), dtype), copy=False)
    k = Tensor(as_dtype(rng.normal(size=(1, KV, T, 64)).astype(np.float32), dtype), copy=False)
    v = Tensor(as_dtype(rng.normal(size=(1, KV, T, 64)).astype(np.float32), dtype), copy=False)
    if mask_kind == "causal":
        host_mask = np.triu(np.full((T, T), -1e4, np.float32), k=1)
    else:
        host_mask = rng.uniform(-4.0, 0.0, size=(T, T)).astype(np.float32)
    mask = Tensor(as_dtype(host_mask.reshape(1, 1, T, T), dtype))
    out = _sdpa_graph(q, k, v, mask, H, dtype)
    program = compile_graph(out, compiler="hip", dynamic_inputs=(q, k, v))
    sdpa_steps = [s for s in program._planned.steps if s.attrs.get("divisor") is not None]
    assert len(sdpa_steps) == 1
    assert (sdpa_steps[0].attrs["causal"] is not None) == (mask_kind == "causal")
    (got,) = program()
    (expected,) = realize(out, compiler="cpu")
    tolerance = 1e-2 if dtype == np.float16 else 3e-2
    np.testing.assert_allclose(as_float(got), as_float(expected), rtol=tolerance, atol=tolerance)


def test_empty_tensors(hip):
    announce("empty tensors")
    empty = Tensor(np.empty((0, 4), dtype=np.float32))
    assert empty.softmax(axis=-1).numpy(compiler="hip").shape == (0, 4)
    assert (empty * 2.0).numpy(compiler="hip").shape == (0, 4)
    np.testing.assert_allclose(empty.sum(axis=0).numpy(compiler="hip"), np.zeros(4))


def test_float64_is_rejected(hip):
    announce("float64 rejected")
    with pytest.raises(TypeError):
        (Tensor([1.0, 2.0]) * 2.0).numpy(compiler="hip")


def test_safetensors_loading(hip, tmp_path):
    announce("safetensors")
    import json
    import struct

    weights = {"a": np.arange(6, dtype=np.float32).reshape(2, 3), "b": np.ones(4, np.float16)}
    header, blobs, offset = {}, [], 0
    for name, value in weights.items():
        raw = value.tobytes()
        header[name] = {"dtype": {"float32": "F32", "float16": "F16"}[value.dtype.name],
                        "shape": list(value.shape), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    blob = json.dumps(header).encode()
    path = tmp_path / "w.safetensors"
    path.write_bytes(struct.pack("<Q", len(blob)) + blob + b"".join(blobs))
    from chomikgrad.llama import load_safetensors

    loaded = load_safetensors(path, hip.device, dtype=np.float16)
    assert loaded["a"].dtype == np.float16 and loaded["a"].shape == (2, 3)
    np.testing.assert_array_equal(loaded["a"].numpy(compiler="hip"), weights["a"].astype(np.float16))
    bf = load_safetensors(path, hip.device, dtype=BFLOAT16)
    np.testing.assert_array_equal(bf["b"].numpy(compiler="hip").view(np.uint16),
                                  to_bf16(np.ones(4, np.float32)).view(np.uint16))


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("S", [12, 200])
def test_prefill_gemm_epilogues_match_oracle(hip, dtype, S):
    """A 16-bit prefill layer through the MFMA GEMM with its fused epilogues:
    gate/up as one GEMM with the SiLU product, o_proj and down_proj adding
    the residual (FFN width 688 leaves ragged output tiles)."""
    from chomikgrad import synthetic
    from chomikgrad._planner import K_ELEMENTWISE, K_GEMM
    from chomikgrad.llama import LlamaConfig, LlamaForCausalLM, position_selector

    announce(f"prefill GEMM epilogues {dtype_name(dtype)} S={S}")
    config = LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=688, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    weights = synthetic.weights_as_tensors(synthetic.host_weights(config, dtype, seed=11))
    model = LlamaForCausalLM(config, weights, sequence_length=S, cache_length=S, dtype=dtype)
    tokens = Tensor(np.random.default_rng(S).integers(0, 128, (1, S)).astype(np.int32), copy=False)
    outputs = model.prefill(tokens, Tensor(position_selector(S - 1, S, dtype=dtype)))
    program = compile_graph(*outputs, compiler="hip", dynamic_inputs=(tokens,))
    gemms = [s for s in program._planned.steps if s.kind == K_GEMM]
    assert sum(g.attrs.get("up") is not None for g in gemms) == 1
    assert sum(g.attrs.get("res") is not None for g in gemms) == 2
    assert not any(s.kind == K_ELEMENTWISE for s in program._planned.steps)
    got = program()
    expected = realize(*outputs, compiler="cpu")
    for value, reference in zip(got, expected):
        np.testing.assert_allclose(as_float(value), as_float(reference), rtol=2e-2, atol=3e-2)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
def test_gemm_8_wave_tiles_with_epilogues(hip, dtype):
    """The 8-wave GEMM tiles with their fused epilogues: the SiLU pair over
    512 tiles of 256 x 128 (gate and up rows interleaved per fragment) and
    the residual epilogue over 256 tiles of 128 x 128 (the last row of tiles
    ragged), against float32 products of the same rounded inputs with the
    portable graph's rounding points."""
    from chomikgrad._planner import K_GEMM

    announce(f"gemm 8-wave tiles with epilogues {dtype_name(dtype)}")
    rng = np.random.default_rng(5)
    K = 192

    def rounded(values):
        return as_float(as_dtype(np.asarray(values, np.float32), dtype))

    x1 = as_dtype(rng.normal(size=(1, 1024, K)).astype(np.float32), dtype)
    wg = as_dtype((rng.normal(size=(8192, K)) * 0.05).astype(np.float32), dtype)
    wu = as_dtype((rng.normal(size=(8192, K)) * 0.05).astype(np.float32), dtype)
    x2 = as_dtype(rng.normal(size=(1, 1960, K)).astype(np.float32), dtype)
    wo = as_dtype((rng.normal(size=(2048, K)) * 0.05).astype(np.float32), dtype)
    h = as_dtype(rng.normal(size=(1, 1960, 2048)).astype(np.float32), dtype)
    X1, WG, WU, X2, WO, Hh = (Tensor(v) for v in (x1, wg, wu, x2, wo, h))
    gate = X1 @ WG.T
    act = gate / (1 + (-gate).exp()) * (X1 @ WU.T)
    res = Hh + X2 @ WO.T
    program = compile_graph(act, res, compiler="hip")
    gemms = [st for st in program._planned.steps if st.kind == K_GEMM]
    assert len(gemms) == 2 and sum(g.attrs.get("up") is not None for g in gemms) == 1
    got_act, got_res = program()
    g = rounded(as_float(x1)[0] @ as_float(wg).T)
    u = rounded(as_float(x1)[0] @ as_float(wu).T)
    denom = rounded(rounded(np.exp(-g)) + 1)
    want_act = rounded(rounded(g / denom) * u)
    want_res = rounded(as_float(h)[0] + rounded(as_float(x2)[0] @ as_float(wo).T))
    tolerance = dict(rtol=1e-2, atol=1e-2) if dtype == np.float16 else dict(rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(as_float(got_act).reshape(want_act.shape), want_act, **tolerance)
    np.testing.assert_allclose(as_float(got_res).reshape(want_res.shape), want_res, **tolerance)


def test_safetensors_bf16_stored_tensor_on_device(hip, tmp_path):
    """A BF16-stored tensor uploaded as bfloat16 (bits unchanged) and as
    float32 (exact widening), read back through the adapter."""
    announce("safetensors BF16-stored tensor")
    from test_host_cpu import BF16_BITS, BF16_VALUES, write_safetensors

    path = tmp_path / "bf.safetensors"
    write_safetensors(path, {"w": ("BF16", (8,), BF16_BITS.tobytes())})
    native = hip.device.load_safetensors(path)
    assert hip.device.dtype(native["w"]) == BFLOAT16
    np.testing.assert_array_equal(hip.device.to_numpy(native["w"]).view(np.uint16), BF16_BITS)
    wide = hip.device.load_safetensors(path, dtype=np.float32)
    np.testing.assert_array_equal(hip.device.to_numpy(wide["w"]), BF16_VALUES)


def test_top_k_sampling_matches_oracle_runtime(hip):
    """Seeded temperature/top-k generation (generate_tinyllama.py:124-143) on
    the C1 model: the hip runtime copies each logits row to the host
    (HIPDeviceAdapter.to_numpy) and samples with the same generator as the
    oracle runtime, so the two draw the same tokens (their float32 logits
    agree to ~1e-6, far inside any sampling interval of these draws)."""
    announce("top-k sampling, C1 model, hip vs oracle")
    from chomikgrad import synthetic
    from chomikgrad.runtime import LlamaRuntime

    spec = synthetic.TINY
    weights = synthetic.weights_as_tensors(synthetic.host_weights(spec.config, spec.dtype, seed=0))
    prompt = synthetic.prompt_ids(spec.config.vocab_size, 16, 0)
    results = {}
    for name in ("hip", "cpu"):
        runtime = LlamaRuntime(spec.config, weights, compiler=name, dtype=spec.dtype)
        results[name] = runtime.generate(prompt, 24, temperature=0.8, top_k=20, seed=5)
    assert results["hip"]["generated_token_ids"] == results["cpu"]["generated_token_ids"]
    greedy = LlamaRuntime(spec.config, weights, compiler="hip", dtype=spec.dtype).generate(prompt, 24)
    assert greedy["generated_token_ids"] != results["hip"]["generated_token_ids"]  # sampling took effect
