"""Llama graphs on the hip plugin against the reference's golden vectors and
the oracle: C1 end to end, float16 TinyLlama-shape parity, the lowered
graph against the portable CPU graph (the reference's tests/test_mlx.py
template), block verification, batched bf16 decode, and the resident loop."""

from __future__ import annotations

import numpy as np
import pytest

from chomikgrad import Tensor, compile_graph, realize, synthetic
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
from chomikgrad.runtime import LlamaRuntime
from conftest import GOLDEN, tiny_weights

pytestmark = pytest.mark.gpu

FP16_ATOL, FP16_RTOL = 2e-2, 1e-2


def announce(name):
    print(f"[gpu case] {name}", flush=True)


def recording_runtime(runtime):
    rows = []
    device = runtime.device
    original = device.argmax

    def record(value):
        rows.append(np.asarray(device.to_numpy(value)).reshape(-1).copy())
        return original(value)

    device.argmax = record
    return rows, lambda: setattr(device, "argmax", original)


@pytest.mark.parametrize("loop", ["reference", "resident"])
def test_c1_greedy_tokens_and_logits_match_reference(hip, loop):
    announce(f"C1 golden, {loop} loop")
    golden = np.load(GOLDEN / "c1_greedy.npz")
    spec = synthetic.TINY
    host = synthetic.host_weights(spec.config, spec.dtype, seed=0)
    runtime = LlamaRuntime(spec.config, synthetic.weights_as_tensors(host), compiler="hip", dtype=spec.dtype)
    rows, restore = recording_runtime(runtime)
    try:
        result = runtime.generate(golden["prompt"], 32, loop=loop)
    finally:
        restore()
    assert result["generated_token_ids"] == golden["tokens"].tolist()
    if loop == "reference":
        np.testing.assert_allclose(np.stack(rows), golden["logits"], rtol=1e-4, atol=1e-5)


def test_fp16_layer_matches_reference_golden(hip):
    announce("fp16 TinyLlama-shape layer golden")
    golden = np.load(GOLDEN / "fp16_step.npz")
    config = synthetic._cfg(1024, 2048, 5632, 1, 32, 4)
    host = synthetic.host_weights(config, np.float16, seed=3)
    runtime = LlamaRuntime(config, synthetic.weights_as_tensors(host), compiler="hip", dtype=np.float16)
    rows, restore = recording_runtime(runtime)
    try:
        result = runtime.generate(golden["prompt"], 5, loop="reference")
    finally:
        restore()
    assert result["generated_token_ids"] == golden["tokens"].tolist()
    np.testing.assert_allclose(np.stack(rows).astype(np.float32), golden["logits"].astype(np.float32),
                               atol=FP16_ATOL, rtol=FP16_RTOL)


def test_c2_tinyllama_fp16_greedy_matches_oracle_fixture(hip):
    path = GOLDEN / "c2_fp16_greedy.npz"
    if not path.exists():
        pytest.skip("c2 fixture not generated")
    announce("C2 TinyLlama fp16, 32-token prompt, 32 greedy steps")
    golden = np.load(path)
    spec = synthetic.TINYLLAMA
    host = synthetic.host_weights(spec.config, spec.dtype, seed=0)
    runtime = LlamaRuntime(spec.config, synthetic.weights_as_tensors(host), compiler="hip", dtype=spec.dtype)
    rows, restore = recording_runtime(runtime)
    try:
        reference_loop = runtime.generate(golden["prompt"], 32, loop="reference")
    finally:
        restore()
    assert reference_loop["generated_token_ids"] == golden["tokens"].tolist()
    np.testing.assert_allclose(np.stack(rows).astype(np.float32), golden["logits"].astype(np.float32),
                               atol=FP16_ATOL, rtol=FP16_RTOL)
    resident = runtime.generate(golden["prompt"], 32, loop="resident")
    assert resident["generated_token_ids"] == golden["tokens"].tolist()


def test_llama_lowerings_match_portable_cpu_graph(hip):
    announce("lowered llama vs portable graph")
    config = LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    weights = tiny_weights(config, 23)
    model = LlamaForCausalLM(config, weights, sequence_length=7, dtype=np.float32)
    output = model(Tensor(np.array([[1, 3, 4, 9, 2, 2, 5]], dtype=np.int32), copy=False),
                   Tensor(position_selector(6, 7, dtype=np.float32), copy=False))
    program = compile_graph(output, compiler="hip")
    for name in ("gather", "rms_norm", "rope", "sdpa"):
        assert name in program.source, name
    assert "sqrt" not in program.source
    np.testing.assert_allclose(program()[0], output.numpy(compiler="cpu"), rtol=2e-4, atol=2e-5)


def test_prefill_caches_and_block_verify_match_oracle(hip):
    announce("prefill caches + block verify")
    config = synthetic.TINY.config
    weights = tiny_weights(config, 31)
    prompt, proposed = [5, 9, 1, 33, 7], [2, 40, 11]
    C = 10
    model = LlamaForCausalLM(config, weights, sequence_length=len(prompt), cache_length=C, dtype=np.float32)
    tokens = Tensor(np.asarray([prompt], np.int32), copy=False)
    selector = Tensor(position_selector(len(prompt) - 1, len(prompt), dtype=np.float32))
    got, expected = realize(*model.prefill(tokens, selector), compiler="hip"), realize(
        *model.prefill(tokens, selector), compiler="cpu")
    for g, e in zip(got, expected):
        np.testing.assert_allclose(g, e, rtol=1e-4, atol=1e-5)
    caches = [Tensor(c) for c in expected[1:]]
    n, position = len(proposed), len(prompt)
    placement, write, attention = block_masks(position, n, C, np.float32)
    block = LlamaDecoderBlock(config, weights, block_length=n, cache_length=C, dtype=np.float32)
    leaves = [Tensor(np.asarray([proposed], np.int32), copy=False),
              Tensor(_rope_rotations(n, config.head_size, config.rope_theta, np.float32, offset=position)),
              Tensor(attention), Tensor(placement), Tensor(write), Tensor(np.asarray(position, np.int32))]
    outputs = block(*leaves[:5], list(zip(caches[::2], caches[1::2])), position=leaves[5])
    got, expected = realize(*outputs, compiler="hip"), realize(*outputs, compiler="cpu")
    for g, e in zip(got, expected):
        np.testing.assert_allclose(g, e, rtol=1e-4, atol=1e-5)


def test_batched_bf16_decode_matches_emulated_oracle(hip):
    announce("batched bf16 decode")
    config = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128,
                         rope_theta=500_000.0)
    host = synthetic.host_weights(config, BFLOAT16, seed=3, tie_embeddings=True)
    weights = synthetic.weights_as_tensors(host)
    B, C = 4, 32
    positions = np.array([4, 30, 2, 17], np.int32)
    rng = np.random.default_rng(6)
    caches = [Tensor(to_bf16(rng.normal(size=(B, 2, C, 64)) * 0.3), copy=False) for _ in range(4)]
    attention = np.concatenate([decode_masks(int(p), C, np.float32)[0] for p in positions]).reshape(B, 1, 1, C)
    write = np.concatenate([decode_masks(int(p), C, np.float32)[1] for p in positions]).reshape(B, 1, C, 1)
    rotation = np.concatenate([_rope_rotations(1, 64, config.rope_theta, np.float32, offset=int(p))
                               for p in positions]).reshape(B, 1, 1, 64, 64)
    leaves = [Tensor(np.array([[1], [7], [200], [511]], np.int32), copy=False),
              Tensor(to_bf16(rotation), copy=False), Tensor(to_bf16(attention), copy=False),
              Tensor(to_bf16(write), copy=False), Tensor(positions, copy=False)]
    dec = LlamaBatchedDecoderStep(config, weights, batch=B, cache_length=C, dtype=BFLOAT16)
    outputs = dec(*leaves[:4], list(zip(caches[::2], caches[1::2])), position=leaves[4])
    got, expected = realize(*outputs, compiler="hip"), realize(*outputs, compiler="cpu")
    np.testing.assert_allclose(bf16_to_float32(got[0]), bf16_to_float32(expected[0]), atol=3e-2, rtol=3e-2)
    for g, e in zip(got[1:], expected[1:]):
        np.testing.assert_allclose(bf16_to_float32(g), bf16_to_float32(e), atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
def test_attention_partials_combined_by_output_projection(hip, dtype, monkeypatch):
    """Batch-1 decode layer with 16 heads of 64 over a 100-row cache (4
    chunks): the attention stores partials only and the output projection
    (K_ATTN_PROJ) combines them; the same layer with the fusion off combines
    in the attention.  Both match the oracle; the caches are exact; the two
    hip programs agree to the last bit (the same combine and row-GEMV
    arithmetic)."""
    from chomikgrad import _planner

    announce(f"attention partials combined by the output projection {np.dtype(dtype).name}")
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
    got = {}
    for fuse in (1, 0):
        monkeypatch.setattr(_planner, "ATTN_PROJ_FUSE", fuse)
        hip.close()  # drop programs cached by signature: plan again with the knob
        program = compile_graph(*outputs, compiler="hip")
        assert ("attn_proj" in program.source) == bool(fuse)
        values = [hip.device.to_numpy(v) for v in program.run(synchronize=True)]
        as_float = (lambda v: bf16_to_float32(v)) if dtype is BFLOAT16 else (lambda v: np.asarray(v, np.float32))
        np.testing.assert_allclose(as_float(values[0]), as_float(expected[0]), atol=FP16_ATOL, rtol=FP16_RTOL)
        for value, reference in zip(values[1:], expected[1:]):
            np.testing.assert_array_equal(np.asarray(value).view(np.uint8), np.asarray(reference).view(np.uint8))
        got[fuse] = values[0]
    np.testing.assert_array_equal(np.asarray(got[1]).view(np.uint8), np.asarray(got[0]).view(np.uint8))
