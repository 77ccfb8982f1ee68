"""The hip plugin's planner on CPU: lowering choice, fusion passes, memory
plan and tape encoding, executed by the host tape model (tests/tape_model.py)
and compared with the oracle.  No GPU is involved; the GPU tests repeat the
same cases through libchomik_hip.so."""

from __future__ import annotations

import numpy as np
import pytest

from chomikgrad import Tensor, realize, synthetic
from chomikgrad._planner import (K_DECODE_ATTN, K_ELEMENTWISE, K_FILL, K_GEMM, K_GEMV, K_KV_PLACE, K_KV_WRITE, K_MATMUL,
                                 K_SDPA, plan_graph)
from chomikgrad.dtypes import BFLOAT16, bf16_to_float32, to_bf16
from chomikgrad.llama import (
    LlamaBatchedDecoderStep,
    LlamaConfig,
    LlamaDecoderBlock,
    LlamaDecoderStep,
    LlamaForCausalLM,
    _rope_rotations,
    block_masks,
    decode_masks,
    position_selector,
)
from conftest import tiny_weights
import attention_cases
from tape_model import CpuPlanCompiler, run

COMPILER = CpuPlanCompiler()


def model_run(outputs, dynamic=(), donate=(), bindings=None):
    nodes = [t._node for t in outputs]
    planned = plan_graph(COMPILER, nodes, [t._node for t in dynamic], [t._node for t in donate])
    values = {}
    for leaf in planned.input_slots:
        values[leaf] = (bindings or {}).get(leaf, leaf.numpy_value() if leaf.value is not None else None)
    return planned, run(planned, values)


def as_float(values):
    values = np.asarray(values)
    return bf16_to_float32(values) if values.dtype == BFLOAT16 else values.astype(np.float32)


def test_six_ops_and_gather_match_oracle():
    left = Tensor([[1.0, -2.0, 0.5], [3.0, 4.0, -1.0]], dtype=np.float32)
    right = Tensor([[2.0, 1.0], [-1.0, 0.5], [3.0, -2.0]], dtype=np.float32)
    result = ((left @ right).relu() + 0.25).permute(1, 0).reshape(1, 4).sum(axis=1)
    planned, got = model_run([result])
    np.testing.assert_allclose(got[0], result.numpy(compiler="cpu"), rtol=1e-5, atol=1e-6)
    assert "fused_elementwise" in planned.source and "matmul" in planned.source
    table = Tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dtype=np.float32)
    ids = Tensor(np.array([[2, 0, -1]], dtype=np.int32), copy=False)
    _, got = model_run([table.gather(ids)])
    np.testing.assert_allclose(got[0], [[[5.0, 6.0], [1.0, 2.0], [5.0, 6.0]]])


def test_gather_out_of_range_raises():
    table = Tensor([[1.0, 2.0]], dtype=np.float32)
    with pytest.raises(IndexError):
        model_run([table.gather(Tensor(np.array([1], dtype=np.int32)))])


@pytest.mark.parametrize("dtype", [np.float32, np.float16, BFLOAT16])
def test_batched_and_broadcast_matmul(dtype):
    rng = np.random.default_rng(19)
    left = Tensor(rng.normal(size=(2, 4, 3, 5)).astype(np.float32), dtype=dtype)
    right = Tensor(rng.normal(size=(2, 4, 5, 6)).astype(np.float32), dtype=dtype)
    weight = Tensor(rng.normal(size=(5, 7)).astype(np.float32), dtype=dtype)
    outputs = [left @ right, left @ weight, (left.transpose(-2, -1).transpose(-2, -1)) @ right]
    _, got = model_run(outputs)
    for out, value in zip(outputs, got):
        np.testing.assert_allclose(as_float(value), as_float(out.numpy(compiler="cpu")), rtol=1e-2, atol=1e-2)


def test_softmax_reductions_and_elementwise_chains():
    rng = np.random.default_rng(29)
    source = Tensor(rng.normal(size=(2, 3, 4)).astype(np.float16))
    outputs = [source.softmax(axis=1), source.softmax(axis=-1), source.max(axis=(0, 2), keepdims=True),
               (source.exp() * 2.0 - source.sqrt()).mean(axis=-1), source.log_softmax(axis=-1)]
    _, got = model_run(outputs)
    for out, value in zip(outputs, got):
        expected = out.numpy(compiler="cpu")
        np.testing.assert_allclose(value.astype(np.float32), expected.astype(np.float32),
                                   rtol=2e-3, atol=2e-3, equal_nan=True)


def test_linear_uses_gemv_with_fusions():
    config = synthetic.TINY.config
    weights = tiny_weights(config, 1)
    C = 20
    position = 7
    dec = LlamaDecoderStep(config, weights, cache_length=C, dtype=np.float32)
    attention, write = decode_masks(position, C, np.float32)
    leaves = [Tensor(np.array([[5]], np.int32), copy=False),
              Tensor(_rope_rotations(1, 64, config.rope_theta, np.float32, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    rng = np.random.default_rng(2)
    caches = [Tensor(rng.normal(size=(1, 2, C, 64)).astype(np.float32), copy=False) for _ in range(4)]
    outputs = dec(*leaves[:4], list(zip(caches[::2], caches[1::2])), position=leaves[4])
    expected = realize(*outputs, compiler="cpu")
    planned, got = model_run(outputs, leaves + caches, donate=caches)
    kinds = [s.kind for s in planned.steps]
    assert kinds.count(K_GEMV) == 4 * config.num_hidden_layers + 1
    assert kinds.count(K_DECODE_ATTN) == config.num_hidden_layers
    assert kinds.count(K_KV_WRITE) == 0 and kinds.count(K_SDPA) == 0
    assert len(kinds) == 5 * config.num_hidden_layers + 2  # gather + per layer 5 + lm_head
    assert "gemv[rms_norm]" in planned.source and "gemv[rms_norm+silu_mul]" in planned.source
    assert "gemv[residual]" in planned.source
    for value, reference in zip(got, expected):
        np.testing.assert_allclose(value, reference, rtol=1e-4, atol=1e-5)
    # Donated caches are updated in place: the outputs are the input leaves.
    assert [spec[0] for spec in planned.output_specs[1:]] == ["input"] * 4


def _fp16_layer():
    config = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1408, num_hidden_layers=1,
                         num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=256)
    host = synthetic.host_weights(config, np.float16, seed=7)
    return config, synthetic.weights_as_tensors(host)


def test_fp16_decode_step_matches_oracle_roundings():
    config, weights = _fp16_layer()
    C, position = 24, 11
    rng = np.random.default_rng(4)
    caches = [Tensor((rng.normal(size=(1, 2, C, 64)) * 0.5).astype(np.float16), copy=False) for _ in range(2)]
    attention, write = decode_masks(position, C, np.float16)
    leaves = [Tensor(np.array([[17]], np.int32), copy=False),
              Tensor(_rope_rotations(1, 64, config.rope_theta, np.float16, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    dec = LlamaDecoderStep(config, weights, cache_length=C, dtype=np.float16)
    outputs = dec(*leaves[:4], [(caches[0], caches[1])], position=leaves[4])
    expected = realize(*outputs, compiler="cpu")
    _, got = model_run(outputs, leaves + caches)
    # The fused kernels round where the portable graph rounds, except the
    # decode attention's softmax and P V, which run in float32 and round once;
    # the order of float32 sums differs too.  The logits stay within a few
    # float16 ulps; the cache rows (RoPE and the blended write) stay exact.
    np.testing.assert_allclose(got[0].astype(np.float32), expected[0].astype(np.float32), atol=2e-3, rtol=2e-3)
    for value, reference in zip(got[1:], expected[1:]):
        np.testing.assert_allclose(value.astype(np.float32), reference.astype(np.float32), atol=2e-3, rtol=1e-2)
        assert np.mean(value == reference) > 0.99


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16])
def test_attention_partials_combined_by_output_projection(dtype, monkeypatch):
    """Batch-1 decode with 16 heads of 64 over a 100-row cache (4 chunks):
    the attention stores its partials only and the output projection
    combines them (K_ATTN_PROJ, residual epilogue); with the fusion off the
    attention combines itself.  Both match the oracle's portable graph."""
    from chomikgrad import _planner

    config = LlamaConfig(vocab_size=256, hidden_size=1024, intermediate_size=512, num_hidden_layers=1,
                         num_attention_heads=16, num_key_value_heads=4, max_position_embeddings=128)
    weights = synthetic.weights_as_tensors(synthetic.host_weights(config, dtype, seed=11))
    C, position = 100, 77
    rng = np.random.default_rng(8)
    caches = [Tensor((rng.normal(size=(1, 4, C, 64)) * 0.5).astype(np.float32), dtype=dtype) for _ in range(2)]
    attention, write = decode_masks(position, C, dtype)
    leaves = [Tensor(np.array([[17]], np.int32), copy=False),
              Tensor(_rope_rotations(1, 64, config.rope_theta, dtype, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    dec = LlamaDecoderStep(config, weights, cache_length=C, dtype=dtype)
    outputs = dec(*leaves[:4], [(caches[0], caches[1])], position=leaves[4])
    expected = realize(*outputs, compiler="cpu")
    results = {}
    for fuse in (1, 0):
        monkeypatch.setattr(_planner, "ATTN_PROJ_FUSE", fuse)
        planned, got = model_run(outputs, leaves + caches)
        kinds = [s.kind for s in planned.steps]
        assert kinds.count(_planner.K_ATTN_PROJ) == fuse
        attn = next(s for s in planned.steps if s.kind == K_DECODE_ATTN)
        assert bool(attn.attrs.get("partials_only")) == bool(fuse)
        np.testing.assert_allclose(as_float(got[0]), as_float(expected[0]), atol=2e-2, rtol=1e-2)
        for value, reference in zip(got[1:], expected[1:]):  # the caches: exact
            np.testing.assert_array_equal(np.asarray(value).view(np.uint8), np.asarray(reference).view(np.uint8))
        results[fuse] = got[0]
    # the fused projection computes the same values as the unfused chain
    np.testing.assert_allclose(as_float(results[1]), as_float(results[0]), atol=1e-2, rtol=1e-2)


def test_prefill_with_cache_placement():
    config = synthetic.TINY.config
    weights = tiny_weights(config, 9)
    model = LlamaForCausalLM(config, weights, sequence_length=6, cache_length=10, dtype=np.float32)
    tokens = Tensor(np.array([[1, 5, 9, 2, 4, 3]], np.int32), copy=False)
    outputs = model.prefill(tokens, Tensor(position_selector(5, 6, dtype=np.float32)))
    expected = realize(*outputs, compiler="cpu")
    _, got = model_run(outputs, [tokens])
    for value, reference in zip(got, expected):
        np.testing.assert_allclose(value, reference, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("cache_length", [16, 12], ids=["cache16", "cache12"])
@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
def test_half_precision_prefill_uses_mfma_gemm(dtype, cache_length):
    """Prefill linears of a 16-bit model with more than 8 rows become K_GEMM
    steps (row-major activations times W^T, fp32 accumulation, one rounding):
    the tape model of those steps matches the oracle's np.matmul.  A cache
    as long as the prompt is placed by the copy alone (no zero fill)."""
    config = LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=688, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    host = synthetic.host_weights(config, dtype, seed=11)
    weights = synthetic.weights_as_tensors(host)
    S = 12
    model = LlamaForCausalLM(config, weights, sequence_length=S, cache_length=cache_length, dtype=dtype)
    ids = np.random.default_rng(4).integers(0, 128, (1, S)).astype(np.int32)
    tokens = Tensor(ids, copy=False)
    outputs = model.prefill(tokens, Tensor(position_selector(S - 1, S, dtype=dtype)))
    expected = realize(*outputs, compiler="cpu")
    planned, got = model_run(outputs, [tokens])
    gemms = [s for s in planned.steps if s.kind == K_GEMM]
    assert len(gemms) == 4  # q|k|v (one launch), o (+ residual), gate/up (+ SiLU), down (+ residual)
    assert sum(len(g.attrs.get("segments") or ()) == 3 for g in gemms) == 1
    assert sum(g.attrs.get("up") is not None for g in gemms) == 1
    assert sum(g.attrs.get("res") is not None for g in gemms) == 2
    assert not any(s.kind == K_ELEMENTWISE for s in planned.steps)
    # the cache placements K^T @ eye(S, C) become fill + strided copy (the
    # copy alone when S == C); the last-row selector (a one-hot constant) is
    # a row copy: no generic matmul left
    assert sum(s.kind == K_FILL for s in planned.steps) == (2 if cache_length > S else 0)
    assert sum(s.kind == K_MATMUL for s in planned.steps) == 0
    for value, reference in zip(got, expected):
        v, r = np.asarray(value), np.asarray(reference)
        if dtype is BFLOAT16:
            v, r = bf16_to_float32(v), bf16_to_float32(r)
        np.testing.assert_allclose(v.astype(np.float32), r.astype(np.float32), rtol=1e-2, atol=2e-2)


def test_block_verify_uses_kv_place():
    config = synthetic.TINY.config
    weights = tiny_weights(config, 10)
    C, position, n = 12, 6, 3
    rng = np.random.default_rng(1)
    caches = [Tensor(rng.normal(size=(1, 2, C, 64)).astype(np.float32), copy=False) for _ in range(4)]
    placement, write, attention = block_masks(position, n, C, np.float32)
    block = LlamaDecoderBlock(config, weights, block_length=n, cache_length=C, dtype=np.float32)
    leaves = [Tensor(np.array([[3, 8, 1]], np.int32), copy=False),
              Tensor(_rope_rotations(n, 64, config.rope_theta, np.float32, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(placement, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    outputs = block(*leaves[:5], list(zip(caches[::2], caches[1::2])), position=leaves[5])
    expected = realize(*outputs, compiler="cpu")
    planned, got = model_run(outputs, leaves + caches, donate=caches)
    assert any(s.kind == K_KV_PLACE for s in planned.steps)
    for value, reference in zip(got, expected):
        np.testing.assert_allclose(value, reference, rtol=1e-4, atol=1e-5)


def test_batched_bf16_decode():
    config = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                         rope_theta=500_000.0)
    host = synthetic.host_weights(config, BFLOAT16, seed=3, tie_embeddings=True)
    weights = synthetic.weights_as_tensors(host)
    B, C = 3, 16
    positions = np.array([4, 9, 2], np.int32)
    rng = np.random.default_rng(6)
    caches = [Tensor(to_bf16(rng.normal(size=(B, 2, C, 64)) * 0.3), copy=False) for _ in range(2)]
    attention = np.concatenate([decode_masks(int(p), C, np.float32)[0] for p in positions]).reshape(B, 1, 1, C)
    write = np.concatenate([decode_masks(int(p), C, np.float32)[1] for p in positions]).reshape(B, 1, C, 1)
    rotation = np.concatenate([_rope_rotations(1, 64, config.rope_theta, np.float32, offset=int(p))
                               for p in positions]).reshape(B, 1, 1, 64, 64)
    leaves = [Tensor(np.array([[1], [7], [200]], np.int32), copy=False),
              Tensor(to_bf16(rotation), copy=False), Tensor(to_bf16(attention), copy=False),
              Tensor(to_bf16(write), copy=False), Tensor(positions, copy=False)]
    dec = LlamaBatchedDecoderStep(config, weights, batch=B, cache_length=C, dtype=BFLOAT16)
    outputs = dec(*leaves[:4], [(caches[0], caches[1])], position=leaves[4])
    expected = realize(*outputs, compiler="cpu")
    planned, got = model_run(outputs, leaves + caches)
    # every RMSNorm (q/k/v, gate/up, final) is the prologue of a batch GEMV
    assert planned.source.count("gemv[rms_norm") == 3 and " rms_norm(" not in planned.source
    np.testing.assert_allclose(as_float(got[0]), as_float(expected[0]), atol=3e-2, rtol=3e-2)
    for value, reference in zip(got[1:], expected[1:]):
        np.testing.assert_allclose(as_float(value), as_float(reference), atol=2e-2, rtol=2e-2)


def test_batch_row_exact_choice_by_merged_launch(monkeypatch):
    """Batch GEMVs (8 independent bf16 rows) go to the row-exact kernels
    when the merged launch is narrow (<= 2048 output rows) or very tall
    (>= 32768) and K <= 2048; the merged q/k/v (3072 rows), a 4096-row
    launch and a K = 4096 projection stay on the MFMA kernel.  Planning only
    (no kernels run); with the pass switched off nothing is row-exact."""
    from chomikgrad import _planner

    rng = np.random.default_rng(11)

    def act(*shape):
        return Tensor(to_bf16(rng.normal(size=shape)), copy=False)

    def weight(n, k):
        return Tensor(to_bf16(rng.normal(size=(n, k)) * 0.05), copy=False)

    def rms(x):
        norm = Tensor(to_bf16(rng.normal(1.0, 0.2, size=x.shape[-1])), copy=False)
        normed = x / ((x * x).mean(axis=-1, keepdims=True) + 1e-5).sqrt() * norm
        normed._node.lowering = ("rms_norm", (x._node, norm._node), 1e-5)
        return normed

    x, x2, a, h, b, d = act(8, 1, 64), act(8, 1, 64), act(8, 1, 64), act(8, 1, 2048), act(8, 1, 64), act(8, 1, 4096)
    normed, normed2 = rms(x), rms(x2)
    outputs = [normed @ weight(2048, 64).T, normed @ weight(512, 64).T, normed @ weight(512, 64).T,  # q/k/v
               h + a @ weight(2048, 64).T,       # o_proj-like: 2048 rows with the residual
               normed2 @ weight(32768, 64).T,    # lm_head-like: 32768 rows
               b @ weight(4096, 64).T,           # 4096 rows
               d @ weight(2048, 4096).T]         # K = 4096
    dynamic = [t._node for t in (x, x2, a, h, b, d)]

    def exact_rows(enabled):
        monkeypatch.setattr(_planner, "GEMV_BATCH_ROW_EXACT", enabled)
        planned = plan_graph(COMPILER, [t._node for t in outputs], dynamic, [])
        gemvs = [st for st in planned.steps if st.kind == K_GEMV]
        assert len(gemvs) == 5  # q/k/v merged into one launch
        return {(sum(seg["w"].shape[0] for seg in st.attrs["segments"]), st.attrs["K"]): bool(st.attrs.get("exact"))
                for st in gemvs}

    assert exact_rows(True) == {(3072, 64): False, (2048, 64): True, (32768, 64): True,
                                (4096, 64): False, (2048, 4096): False}
    assert not any(exact_rows(False).values())


def test_dynamic_inputs_are_validated():
    from chomikgrad.hip_backend import HIPCompiler

    source = Tensor([1.0, 2.0], dtype=np.float32)
    other = Tensor([3.0], dtype=np.float32)
    with pytest.raises(ValueError):
        HIPCompiler.compile(COMPILER, [(source * 2.0)._node], [(source * 3.0)._node])
    with pytest.raises(ValueError):
        HIPCompiler.compile(COMPILER, [(source * 2.0)._node], [other._node])
    with pytest.raises(ValueError):
        HIPCompiler.compile(COMPILER, [], [])


def test_float64_is_rejected():
    with pytest.raises(TypeError):
        plan_graph(COMPILER, [(Tensor([1.0, 2.0]) * 2.0)._node], [])


def test_memory_plan_reuses_the_arena():
    x = Tensor(np.ones((64, 64), np.float32))
    y = x
    for _ in range(8):
        y = (y @ x).relu()
    planned = plan_graph(COMPILER, [y._node], [])
    per_value = 64 * 64 * 4
    assert planned.arena_bytes <= 3 * per_value


@pytest.mark.parametrize("passes", [0, 1, 2, 4, -1, -2])
@pytest.mark.parametrize("case", [c for c in attention_cases.CASES if c.C * c.B <= 1000], ids=lambda c: c.name)
def test_decode_attention_fusion_matches_oracle(case, passes, monkeypatch):
    """The fused decode attention (split over cache chunks, combined by the
    last workgroup; -1 = the streaming kernel; -2 = the MFMA kernel where it
    applies) against the portable chain on the oracle; caches exact."""
    from chomikgrad import _planner

    monkeypatch.setattr(_planner, "DECODE_ATTN_PASSES", passes)
    outputs, dynamic, caches = attention_cases.build(case)
    expected = realize(*outputs, compiler="cpu")
    for donate in ((), caches):
        planned, got = model_run(outputs, dynamic, donate=donate)
        assert [s.kind for s in planned.steps].count(K_DECODE_ATTN) == 1
        np.testing.assert_allclose(as_float(got[0]), as_float(expected[0]), **attention_cases.tolerance(case))
        for value, reference in zip(got[1:], expected[1:]):
            np.testing.assert_array_equal(np.asarray(value).view(np.uint8), np.asarray(reference).view(np.uint8))


@pytest.mark.parametrize("B,KV,C,G,itemsize", [
    (1, 4, 640, 8, 2), (8, 8, 4109, 4, 2), (1, 4, 32768, 8, 2), (2, 2, 70, 2, 4), (1, 1, 1, 1, 2)])
def test_decode_attention_plan_limits(B, KV, C, G, itemsize, monkeypatch):
    """Every plan covers the cache within the combine's 64 ranges per KV
    head; the streaming ranges are whole passes; long caches stream; forced
    to the MFMA kernel, short 16-bit caches go there, and its at most 8
    waves hold every 32-row block."""
    from chomikgrad import _planner

    for forced in (0, -1, -2, 1, 4):
        monkeypatch.setattr(_planner, "DECODE_ATTN_PASSES", forced)
        plan = _planner.decode_attention_plan(B, KV, C, G, itemsize)
        rpp = _planner.decode_attention_rows(itemsize)
        short16 = itemsize == 2 and C <= 768
        assert (plan["passes"] == 8) == (forced == -2 and short16)
        if plan["passes"] == 8:
            assert plan["chunks"] == 1 and 1 <= plan["rows"] <= 3
            assert -(-C // 32) <= 8 * plan["rows"]
            assert plan["rows"] == 1 or -(-C // 32) > 8 * (plan["rows"] - 1)
        elif plan["passes"] == 0:
            assert plan["rows"] % rpp == 0 and plan["unroll"] in (2, 4)
            assert plan["chunks"] == -(-C // plan["rows"])
            assert (plan["chunks"] - 1) * plan["rows"] < C
        else:
            assert plan["chunks"] == -(-C // (rpp * plan["passes"]))
        if forced == 0 and C >= 4096:
            assert plan["passes"] == 0  # long caches always stream
        if forced <= 0:
            assert plan["chunks"] <= _planner.DECODE_ATTN_MAX_CHUNKS


def test_mfma_gemv_block_split_plan():
    """Narrow MFMA GEMVs (a batch of 8 sequences) share each 16-column tile
    among several blocks over K, with one zero-initialised workspace (tickets, then the partial tiles)
    sized for the largest; wide or short-K ones stay unsplit; the planned
    program computes the portable chain's values."""
    from chomikgrad import _planner

    rng = np.random.default_rng(3)
    x = Tensor(rng.normal(size=(8, 1, 8192)).astype(np.float32), dtype=np.float16)
    h = Tensor(rng.normal(size=(8, 1, 384)).astype(np.float32), dtype=np.float16)
    narrow = Tensor((rng.normal(size=(384, 8192)) * 0.02).astype(np.float32), dtype=np.float16)
    wide = Tensor((rng.normal(size=(8192, 2048)) * 0.05).astype(np.float32), dtype=np.float16)
    short = Tensor((rng.normal(size=(384, 256)) * 0.05).astype(np.float32), dtype=np.float16)
    y = Tensor(rng.normal(size=(8, 1, 256)).astype(np.float32), dtype=np.float16)
    z = Tensor(rng.normal(size=(8, 1, 2048)).astype(np.float32), dtype=np.float16)
    outputs = [h + x @ narrow.T, z @ wide.T, y @ short.T]  # distinct inputs: no sibling merge
    planned, got = model_run(outputs)
    gemvs = {s.attrs["segments"][0]["w"].shape: s for s in planned.steps if s.kind == K_GEMV}
    assert gemvs[(384, 8192)].attrs["blocks"] == 4  # 24 tiles, 256 k-steps: 96 blocks of 64 k-steps
    assert "blocks" not in gemvs[(8192, 2048)].attrs and "blocks" not in gemvs[(384, 256)].attrs
    workspace, ticket_bytes = gemvs[(384, 8192)].attrs["workspace"], gemvs[(384, 8192)].attrs["ticket_bytes"]
    assert ticket_bytes == 256  # 24 tickets, 256-byte aligned
    assert workspace.size * 4 >= ticket_bytes + _planner.gemv_partial_bytes(gemvs[(384, 8192)], 4) == 256 + 24 * 4 * 1024
    expected = realize(*outputs, compiler="cpu")
    for value, reference in zip(got, expected):
        np.testing.assert_allclose(np.asarray(value, np.float32), np.asarray(reference, np.float32), rtol=2e-2, atol=2e-2)


def test_transposed_causal_mask_is_not_treated_as_causal():
    """A transposed causal triangle is a view of the same constant with other
    strides and is anti-causal: the planner must read the mask through the
    view and keep it, not drop it as a proved causal mask."""
    from chomikgrad.llama import _tag

    rng = np.random.default_rng(3)
    T, hd = 24, 64
    q, k, v = (Tensor(rng.normal(size=(1, 2, T, hd)).astype(np.float16)) for _ in range(3))
    tri = np.triu(np.full((T, T), -1e4, np.float32), 1).astype(np.float16)[None, None]
    for mask, causal in ((Tensor(tri), True), (Tensor(tri).transpose(-2, -1), False),
                         (Tensor(tri[:, :, ::-1, ::-1].copy()), False)):
        scores = (q @ k.transpose(-2, -1)) / np.sqrt(hd) + mask
        out = _tag(scores.softmax(axis=-1) @ v, "sdpa", (q, k, v, mask), 1 / np.sqrt(hd))
        planned, got = model_run([out], dynamic=[q])  # specialised: the mask is a captured constant
        steps = [s for s in planned.steps if s.kind == K_SDPA]
        assert len(steps) == 1 and (steps[0].attrs["causal"] is not None) == causal
        np.testing.assert_allclose(got[0].astype(np.float32), out.numpy(compiler="cpu").astype(np.float32),
                                   atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
def test_verify_block_plans_row_exact_kernels(dtype, monkeypatch):
    """A verification block (5 positions of one sequence, LlamaDecoderBlock):
    its linears are planned row-exact (the single-token step's arithmetic
    per row, RMSNorm as the prologue) and its attention as the read-only
    decode attention over the placed caches (the decode step's kernel, one
    "sequence" per block row); the tape computes the oracle's values."""
    config = LlamaConfig(vocab_size=300, hidden_size=512, intermediate_size=1376, num_hidden_layers=2,
                         num_attention_heads=8, num_key_value_heads=4, max_position_embeddings=128)
    weights = synthetic.weights_as_tensors(synthetic.host_weights(config, dtype, seed=13))
    C, position, block = 90, 37, 5
    placement, write, attention = block_masks(position, block, C, dtype)
    leaves = [Tensor(np.array([[4, 250, 17, 99, 3]], np.int32), copy=False),
              Tensor(_rope_rotations(block, 64, config.rope_theta, dtype, offset=position), copy=False),
              Tensor(attention, copy=False), Tensor(placement, copy=False), Tensor(write, copy=False),
              Tensor(np.asarray(position, np.int32), copy=False)]
    rng = np.random.default_rng(8)
    caches = [Tensor(as_dtype_host(rng.normal(0, 0.5, (1, 4, C, 64)), dtype), copy=False) for _ in range(4)]
    step = LlamaDecoderBlock(config, weights, block_length=block, cache_length=C, dtype=dtype)
    outputs = step(*leaves[:5], list(zip(caches[::2], caches[1::2])), position=leaves[5])
    expected = realize(*outputs, compiler="cpu")
    planned, got = model_run(outputs, leaves + caches, donate=caches)
    source = planned.source
    assert source.count("decode_attention[block]") == 2 and " sdpa(" not in source
    assert source.count("gemv[rms_norm+row_exact]") == 3  # q/k/v of 2 layers + lm_head
    assert source.count("gemv[rms_norm+silu_mul+row_exact]") == 2
    assert source.count("gemv[residual+row_exact]") == 4
    # rope(k) and both placements of a layer: one paired kv_place
    assert source.count("kv_place[rope+pair]") == 2 and " rope(" not in source and " kv_place(" not in source
    np.testing.assert_allclose(as_float(got[0]), as_float(expected[0]), atol=3e-2, rtol=2e-2)
    for value, reference in zip(got[1:], expected[1:]):
        np.testing.assert_allclose(as_float(value), as_float(reference), atol=3e-2, rtol=2e-2)
    # the fused placement computes what rope + two kv_place steps compute, bit for bit
    from chomikgrad import _planner
    monkeypatch.setattr(_planner, "fuse_block_kv_place", lambda steps, outputs: steps)
    unfused, again = model_run(outputs, leaves + caches, donate=caches)
    assert " rope(" in unfused.source and "kv_place[rope+pair]" not in unfused.source
    for value, reference in zip(got, again):
        assert np.array_equal(np.asarray(value).view(np.uint16), np.asarray(reference).view(np.uint16))


def as_dtype_host(values, dtype):
    from chomikgrad.dtypes import as_dtype
    return as_dtype(np.asarray(values, np.float32), dtype)
