"""The oracle (NumPy ``cpu`` plugin) and the IR, pinned before anything is
compared with them.

Pins, in order of strength:
* golden vectors written by the reference's own cpu plugin
  (tests/golden/make_golden.py): C1's 32 greedy tokens and logits, and a
  TinyLlama-shape float16 layer;
* the reference's own unit tests restated (tests/test_lazy.py,
  tests/test_llama.py, tests/test_generation.py in the reference);
* closed forms and invariants: NumPy's half-precision contraction rule,
  rotate-half RoPE, decode == full forward, block == full forward, and the
  bf16 rounding rule against torch's CPU bfloat16.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from chomikgrad import (
    Compiler,
    GraphPlan,
    LazyNode,
    Op,
    Tensor,
    compile_graph,
    realize,
    register_compiler,
    synthetic,
    verify_greedy_block_with_bonus,
    verify_greedy_candidates,
)
from chomikgrad.dtypes import BFLOAT16, bf16_to_float32, to_bf16
from chomikgrad.llama import (
    LlamaConfig,
    LlamaDecoderBlock,
    LlamaDecoderStep,
    LlamaForCausalLM,
    _rope_rotations,
    block_masks,
    decode_masks,
    load_safetensors,
    position_selector,
    required_weight_shapes,
    token_one_hot,
)
from chomikgrad.runtime import LlamaRuntime
from conftest import GOLDEN, tiny_weights
from oracle import NumpyCompiler, NumpyDeviceAdapter
from oracle.numpy_plugin import _to_bf16

SMALL = LlamaConfig(vocab_size=8, hidden_size=8, intermediate_size=16, num_hidden_layers=2,
                    num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=8)


# ---------------------------------------------------------------- golden vectors
def test_c1_greedy_matches_reference_golden_vectors():
    golden = np.load(GOLDEN / "c1_greedy.npz")
    spec = synthetic.TINY
    host = synthetic.host_weights(spec.config, spec.dtype, seed=0)
    assert synthetic.weights_digest(host) == str(golden["weights_digest"])
    prompt = synthetic.prompt_ids(spec.config.vocab_size, 16, seed=0)
    np.testing.assert_array_equal(prompt, golden["prompt"])
    runtime = LlamaRuntime(spec.config, synthetic.weights_as_tensors(host), compiler="cpu",
                           dtype=spec.dtype)
    rows = []
    original = runtime.device.argmax

    def record(value):
        rows.append(np.asarray(value).reshape(-1).copy())
        return original(value)

    runtime.device.argmax = record
    result = runtime.generate(prompt, 32, loop="reference")
    assert result["generated_token_ids"] == golden["tokens"].tolist()
    np.testing.assert_allclose(np.stack(rows), golden["logits"], rtol=1e-6, atol=1e-7)


def test_fp16_layer_matches_reference_golden_vectors():
    golden = np.load(GOLDEN / "fp16_step.npz")
    config = synthetic._cfg(1024, 2048, 5632, 1, 32, 4)
    host = synthetic.host_weights(config, np.float16, seed=3)
    assert synthetic.weights_digest(host) == str(golden["weights_digest"])
    prompt = synthetic.prompt_ids(config.vocab_size, 8, seed=3)
    runtime = LlamaRuntime(config, synthetic.weights_as_tensors(host), compiler="cpu", dtype=np.float16)
    rows = []
    original = runtime.device.argmax

    def record(value):
        rows.append(np.asarray(value).reshape(-1).copy())
        return original(value)

    runtime.device.argmax = record
    result = runtime.generate(prompt, 5, loop="reference")
    assert result["generated_token_ids"] == golden["tokens"].tolist()
    # Same NumPy calls in the same order: the float16 logits are bit-identical.
    np.testing.assert_array_equal(np.stack(rows), golden["logits"])


# ---------------------------------------------------------------- reference unit tests
class RecordingCompiler(Compiler):
    def __init__(self):
        self.compilations = 0

    def compile(self, outputs, dynamic_inputs=()):
        self.compilations += 1
        return NumpyCompiler().compile(outputs, dynamic_inputs)


def test_graph_is_lazy_and_compiler_is_pluggable():
    recorder = RecordingCompiler()
    register_compiler("test-recording", recorder, replace=True)
    result = (Tensor([1.0, 2.0], dtype=np.float32) + 3.0).relu()
    assert recorder.compilations == 0
    np.testing.assert_allclose(result.numpy(compiler="test-recording"), [4.0, 5.0])
    assert recorder.compilations == 1


def test_cpu_compiler_generates_straight_line_numpy_code():
    output = Tensor([[1.0, 2.0]], dtype=np.float32) @ Tensor([[3.0], [4.0]], dtype=np.float32)
    program = compile_graph(output, compiler="cpu")
    assert "np.matmul" in program.source and "ELEMENTWISE" not in program.source
    np.testing.assert_allclose(program()[0], [[11.0]])


def test_program_run_can_rebind_inputs_without_recompiling():
    source = Tensor([1.0, 2.0], dtype=np.float32)
    program = compile_graph(source * 2.0, compiler="cpu", dynamic_inputs=(source,))
    outputs = program.run({source._node: program.device.array([3.0, 4.0])}, synchronize=False)
    np.testing.assert_allclose(outputs[0], [6.0, 8.0])
    np.testing.assert_allclose(program()[0], [2.0, 4.0])
    assert program.device.name == "cpu" and program.device.argmax(outputs[0]) == 1


def test_instruction_set_has_only_six_operations():
    assert len(Op) == 6


def test_backend_plans_do_not_leak_elementwise_fusions():
    source = Tensor([1.0, -2.0], dtype=np.float32)
    output = ((source + 1.0) * 2.0).relu()
    portable = GraphPlan((output._node,), ())
    nodes = portable.nodes()
    before = tuple(node.lowering for node in nodes)
    fused = GraphPlan((output._node,), {"elementwise_fusion"})
    fused.fuse_elementwise()
    assert fused.lowering(output._node)[0] == "elementwise_fusion"
    assert len(fused.nodes()) < len(nodes)
    assert portable.nodes() == nodes and tuple(n.lowering for n in nodes) == before


def test_gather_forward_known_answer_and_negative_index():
    table = Tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dtype=np.float32)
    ids = Tensor(np.array([[2, 0, 2]], dtype=np.int32), copy=False)
    program = compile_graph(table.gather(ids), compiler="cpu")
    assert "np.take" in program.source
    np.testing.assert_allclose(program()[0], [[[5.0, 6.0], [1.0, 2.0], [5.0, 6.0]]])
    negative = table.gather(Tensor(np.array([-1], dtype=np.int64), copy=False))
    np.testing.assert_allclose(negative.numpy(compiler="cpu"), [[5.0, 6.0]])
    with pytest.raises(IndexError):
        table.gather(Tensor(np.array([3], dtype=np.int32))).numpy(compiler="cpu")


def test_existing_lazy_graph_keeps_pre_assignment_value():
    value = Tensor([2.0], dtype=np.float32)
    old = value * 3.0
    value.assign([5.0])
    np.testing.assert_allclose(old.numpy(compiler="cpu"), [6.0])
    np.testing.assert_allclose((value * 3.0).numpy(compiler="cpu"), [15.0])


def test_copy_false_explicitly_shares_numpy_storage():
    source = np.array([1.0, 2.0], dtype=np.float32)
    shared, owned = Tensor(source, copy=False), Tensor(source)
    source[0] = 9.0
    np.testing.assert_allclose(shared.numpy(compiler="cpu"), [9.0, 2.0])
    np.testing.assert_allclose(owned.numpy(compiler="cpu"), [1.0, 2.0])


def test_token_one_hot_and_position_selector():
    value = token_one_hot([1, 3], 4, 5, fill_token_id=2, dtype=np.float32)
    np.testing.assert_array_equal(value.argmax(axis=-1), [[1, 3, 2, 2]])
    np.testing.assert_array_equal(position_selector(2, 4, dtype=np.float32), [[0, 0, 1, 0]])


def test_rope_rotation_matches_rotate_half():
    value = np.arange(8, dtype=np.float32).reshape(1, 1, 1, 8)
    rotation = _rope_rotations(1, 8, 10_000.0, np.float32)
    np.testing.assert_allclose((value.reshape(1, 1, 1, 1, 8) @ rotation).reshape(value.shape), value)
    rotation = _rope_rotations(2, 8, 10_000.0, np.float32)
    angle = 1 / (10_000.0 ** (np.arange(0, 8, 2) / 8))
    cosine, sine = np.cos(angle), np.sin(angle)
    x = value.reshape(8)
    expected = np.concatenate([x[:4] * cosine - x[4:] * sine, x[4:] * cosine + x[:4] * sine])
    actual = value.reshape(1, 1, 1, 1, 8) @ rotation[:, :, 1:2]
    np.testing.assert_allclose(actual.reshape(8), expected, rtol=1e-6, atol=1e-6)


def test_config_rejects_invalid_grouped_query_attention():
    with pytest.raises(ValueError, match="divisible by KV heads"):
        LlamaConfig(vocab_size=10, hidden_size=24, intermediate_size=48, num_hidden_layers=1,
                    num_attention_heads=6, num_key_value_heads=4, max_position_embeddings=16).validate()


def test_native_tensor_metadata_and_weight_loading():
    marker = object()
    value = Tensor.from_native(marker, backend="test", shape=(2, 3), dtype=np.float32)
    assert value.shape == (2, 3) and value.dtype == np.float32
    assert value._node.native_values["test"] is marker

    class FakeWeightDevice(NumpyDeviceAdapter):
        name = "fake"

        def load_safetensors(self, path):
            return {"weight": np.array([[1.0, 2.0]], dtype=np.float32)}

    weights = load_safetensors(Path("unused.safetensors"), FakeWeightDevice())
    assert weights["weight"].shape == (1, 2) and weights["weight"].dtype == np.float32
    np.testing.assert_array_equal(weights["weight"]._node.native_values["fake"], [[1.0, 2.0]])


def _prefill_caches(weights, prompt, cache_length, config=SMALL):
    model = LlamaForCausalLM(config, weights, sequence_length=len(prompt),
                             cache_length=cache_length, dtype=np.float32)
    native = realize(*model.prefill(Tensor(np.asarray([prompt], dtype=np.int32), copy=False),
                                    Tensor(position_selector(len(prompt) - 1, len(prompt), dtype=np.float32))),
                     compiler="cpu")
    return [(Tensor(native[i]), Tensor(native[i + 1])) for i in range(1, len(native), 2)]


def _full_logits(weights, tokens, config=SMALL):
    full = LlamaForCausalLM(config, weights, sequence_length=len(tokens), dtype=np.float32)
    return full(Tensor(np.asarray([tokens], dtype=np.int32), copy=False),
                Tensor(position_selector(len(tokens) - 1, len(tokens), dtype=np.float32))).numpy(compiler="cpu")


def test_cached_decode_matches_full_causal_forward():
    weights = tiny_weights(SMALL, 4)
    prompt, cache_length, position = [1, 3, 4], 5, 3
    caches = _prefill_caches(weights, prompt, cache_length)
    attention, write = decode_masks(position, cache_length, np.float32)
    decoder = LlamaDecoderStep(SMALL, weights, cache_length=cache_length, dtype=np.float32)
    decoded = realize(*decoder(
        Tensor(token_one_hot([6], 1, 8, fill_token_id=2, dtype=np.float32)),
        Tensor(_rope_rotations(1, SMALL.head_size, SMALL.rope_theta, np.float32, offset=position)),
        Tensor(attention), Tensor(write), caches), compiler="cpu")[0]
    np.testing.assert_allclose(decoded, _full_logits(weights, prompt + [6]), rtol=2e-5, atol=2e-6)


def test_block_decode_matches_each_full_causal_position():
    weights = tiny_weights(SMALL, 14)
    prompt, proposed = [1, 3, 4], [6, 2]
    cache_length = len(prompt) + len(proposed)
    caches = _prefill_caches(weights, prompt, cache_length)
    placement, write, attention = block_masks(3, 2, cache_length, np.float32)
    block = LlamaDecoderBlock(SMALL, weights, block_length=2, cache_length=cache_length, dtype=np.float32)
    actual = realize(*block(
        Tensor(np.asarray([proposed], dtype=np.int32), copy=False),
        Tensor(_rope_rotations(2, SMALL.head_size, SMALL.rope_theta, np.float32, offset=3)),
        Tensor(attention), Tensor(placement), Tensor(write), caches), compiler="cpu")
    for index in range(2):
        np.testing.assert_allclose(actual[0][:, index, :], _full_logits(weights, prompt + proposed[: index + 1]),
                                   rtol=2e-5, atol=2e-6)
    complete = _prefill_caches(weights, prompt + proposed, cache_length)
    flat = [t.numpy(compiler="cpu") for pair in complete for t in pair]
    for block_cache, full_cache in zip(actual[1:], flat):
        np.testing.assert_allclose(block_cache, full_cache, rtol=2e-5, atol=2e-6)


def test_greedy_verification():
    assert verify_greedy_candidates([3, 4, 5], [3, 4, 5]).emitted_tokens == (3, 4, 5)
    result = verify_greedy_candidates([3, 9, 5], [3, 4, 7])
    assert result.emitted_tokens == (3, 4) and result.accepted_draft_tokens == 1
    with pytest.raises(ValueError, match="at least one"):
        verify_greedy_candidates([], [])
    with pytest.raises(ValueError, match="equal lengths"):
        verify_greedy_candidates([1], [1, 2])
    bonus = verify_greedy_block_with_bonus([3, 4], [3, 4, 8])
    assert bonus.emitted_tokens == (3, 4, 8) and bonus.accepted_draft_tokens == 2
    assert verify_greedy_block_with_bonus([3, 9], [3, 4, 8]).emitted_tokens == (3, 4)


# ---------------------------------------------------------------- closed forms
def test_half_precision_contractions_accumulate_in_float32():
    """NumPy's float16 matmul/sum accumulate in float32 and round once: 4096
    ones sum to 4096 (a float16 accumulator would stall at 2048)."""
    ones = Tensor(np.ones((1, 4096), np.float16))
    assert float((ones @ Tensor(np.ones((4096, 1), np.float16))).numpy(compiler="cpu")[0, 0]) == 4096.0
    assert float(ones.sum().numpy(compiler="cpu")) == 4096.0
    rng = np.random.default_rng(0)
    a = rng.normal(size=(1, 2048)).astype(np.float16)
    b = rng.normal(size=(2048, 8)).astype(np.float16)
    expected = (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal((Tensor(a) @ Tensor(b)).numpy(compiler="cpu"), expected)


def test_stable_softmax_known_answer():
    values = Tensor(np.array([1000.0, 1001.0, 999.0], dtype=np.float32)).softmax()
    e = np.exp(np.array([-1.0, 0.0, -2.0]))
    np.testing.assert_allclose(values.numpy(compiler="cpu"), e / e.sum(), rtol=1e-6)


def test_kv_write_is_exact_for_one_hot_masks():
    rng = np.random.default_rng(3)
    cache = rng.normal(size=(1, 2, 6, 4)).astype(np.float16)
    new = rng.normal(size=(1, 2, 1, 4)).astype(np.float16)
    _, write = decode_masks(3, 6, np.float16)
    w = Tensor(write)
    out = (Tensor(cache) * (1 - w) + Tensor(new) * w).numpy(compiler="cpu")
    expected = cache.copy()
    expected[:, :, 3, :] = new[:, :, 0, :]
    np.testing.assert_array_equal(out, expected)


@pytest.mark.parametrize("convert", [_to_bf16, to_bf16])
def test_bf16_rounding_matches_torch(convert):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, 1.0, -1.5, 3.3895314e38, 1e-40, np.inf, -np.inf,
                        1.00390625, 1.01171875, 65504.0], dtype=np.float32)
    values = np.concatenate([rng.normal(size=4096).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 4096),
                             special]).astype(np.float32)
    ours = np.asarray(convert(values)).view(np.uint16)
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    assert np.isnan(bf16_to_float32(to_bf16(np.array([np.nan], np.float32))))[0]


def test_bf16_emulated_ops_round_once_per_op():
    a = to_bf16(np.array([1.0, 3.0], np.float32))
    b = to_bf16(np.array([1.0 / 256, 1.0 / 128], np.float32))
    result = (Tensor(a, dtype=BFLOAT16) + Tensor(b, dtype=BFLOAT16)).numpy(compiler="cpu")
    assert result.dtype == BFLOAT16
    expected = to_bf16(bf16_to_float32(a) + bf16_to_float32(b))
    np.testing.assert_array_equal(result.view(np.uint16), expected.view(np.uint16))

