"""Greedy speculative decoding (the reference's _generate_speculative_loaded,
examples/generate_tinyllama.py:491-622): the emitted sequence must equal the
target's own greedy decoding whatever the draft proposes
(tinyllama_speculative.py:123 in the reference checks exactly that).  The
driver is compiler-agnostic, so these CPU tests run it on the oracle; the
GPU tests repeat it on the hip plugin and at the C5 shapes."""

from __future__ import annotations

import numpy as np
import pytest

from chomikgrad import synthetic
from chomikgrad.dtypes import BFLOAT16, bf16_to_float32
from chomikgrad.llama import LlamaConfig
from chomikgrad.runtime import LlamaRuntime


def tiny_pair(dtype=np.float32):
    target_cfg = LlamaConfig(vocab_size=96, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                             num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    draft_cfg = LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                            num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=128)
    target = synthetic.weights_as_tensors(synthetic.host_weights(target_cfg, dtype, seed=5))
    draft = synthetic.weights_as_tensors(synthetic.host_weights(draft_cfg, dtype, seed=6))
    return target_cfg, target, draft_cfg, draft


@pytest.mark.parametrize("bonus", [False, True], ids=["reference-block", "bonus-block"])
@pytest.mark.parametrize("k", [1, 3])
def test_speculative_equals_greedy_on_oracle(bonus, k):
    target_cfg, target_w, draft_cfg, draft_w = tiny_pair()
    target = LlamaRuntime(target_cfg, target_w, compiler="cpu", dtype=np.float32)
    prompt = [5, 17, 3, 60, 2, 44]
    greedy = target.generate(prompt, 12, loop="reference")["generated_token_ids"]
    for draft_cfg_, draft_w_ in ((draft_cfg, draft_w), (target_cfg, target_w)):
        draft = LlamaRuntime(draft_cfg_, draft_w_, compiler="cpu", dtype=np.float32)
        result = target.generate_speculative(draft, prompt, 12, speculative_tokens=k, bonus=bonus)
        assert result["generated_token_ids"] == greedy
        assert result["proposed_draft_tokens"] >= result["accepted_draft_tokens"] >= 0
    # the target drafting for itself accepts every proposal
    assert result["acceptance_rate"] == 1.0
    rounds = result["target_verification_calls"]
    assert rounds == (-(-11 // (k + 1)) if bonus else -(-11 // k))


def test_speculative_argument_checks():
    target_cfg, target_w, draft_cfg, draft_w = tiny_pair()
    target = LlamaRuntime(target_cfg, target_w, compiler="cpu", dtype=np.float32)
    draft = LlamaRuntime(draft_cfg, draft_w, compiler="cpu", dtype=np.float32)
    with pytest.raises(ValueError):
        target.generate_speculative(draft, [1, 2], 0)
    with pytest.raises(ValueError):
        target.generate_speculative(draft, [1, 2], 4, speculative_tokens=0)
    with pytest.raises(ValueError):
        target.generate_speculative(draft, [], 4)


@pytest.mark.gpu
@pytest.mark.parametrize("loop", ["reference", "resident"])
@pytest.mark.parametrize("bonus", [False, True], ids=["reference-block", "bonus-block"])
def test_speculative_on_hip_matches_oracle_and_greedy(hip, bonus, loop):
    print(f"[gpu case] speculative tiny bonus={bonus} loop={loop}", flush=True)
    target_cfg, target_w, draft_cfg, draft_w = tiny_pair()
    prompt = [5, 17, 3, 60, 2, 44]
    oracle = LlamaRuntime(target_cfg, target_w, compiler="cpu", dtype=np.float32).generate_speculative(
        LlamaRuntime(draft_cfg, draft_w, compiler="cpu", dtype=np.float32), prompt, 12, speculative_tokens=3,
        bonus=bonus)
    target = LlamaRuntime(target_cfg, target_w, compiler="hip", dtype=np.float32)
    draft = LlamaRuntime(draft_cfg, draft_w, compiler="hip", dtype=np.float32)
    got = target.generate_speculative(draft, prompt, 12, speculative_tokens=3, bonus=bonus, loop=loop)
    assert got["loop"].startswith("speculative-resident" if loop == "resident" else "speculative")
    assert got["generated_token_ids"] == oracle["generated_token_ids"]
    assert got["accepted_draft_tokens"] == oracle["accepted_draft_tokens"]
    assert got["generated_token_ids"] == target.generate(prompt, 12, loop="resident")["generated_token_ids"]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [np.float16, BFLOAT16], ids=["fp16", "bf16"])
def test_block_rows_equal_single_token_steps(hip, dtype):
    """Each row of a 5-token verification block equals, bit for bit, the
    single-token decode step at its position fed the same tokens, and the
    caches they leave hold the same values.  The C5 draft's shape (D 512,
    8/4 heads, FFN 1376, vocabulary 32000) covers both GEMV orders (the
    streamed lm_head and the row kernel) and a K that is not an exact fit."""
    print(f"[gpu case] block rows == decode steps, {np.dtype(dtype)}", flush=True)
    spec = synthetic.DRAFT
    weights = synthetic.weights_as_tensors(synthetic.host_weights(spec.config, dtype, seed=4))
    runtime = LlamaRuntime(spec.config, weights, compiler="hip", dtype=dtype)
    prompt = synthetic.prompt_ids(spec.config.vocab_size, 40, seed=4).tolist()
    context, tokens = 120, [31, 7001, 2, 18000, 555]
    _, caches = runtime.prefill(prompt, context)
    rows = []
    for t, token in enumerate(tokens):
        logits, caches = runtime._decode_step(token, len(prompt) + t, context, caches)
        rows.append(np.asarray(hip.device.to_numpy(logits)).reshape(-1))
    _, block_caches = runtime.prefill(prompt, context)
    block_logits, block_caches = runtime._verify_block_logits(tokens, len(prompt), context, block_caches)
    program = runtime._block_programs[(len(tokens), context)][0]
    assert "decode_attention[block]" in program.source and "row_exact" in program.source
    block_rows = np.asarray(hip.device.to_numpy(block_logits)).reshape(len(tokens), -1)
    for t in range(len(tokens)):
        assert np.array_equal(block_rows[t].view(np.uint16), rows[t].view(np.uint16)), f"row {t}"
    for a, b in zip(caches, block_caches):
        assert np.array_equal(as_float(hip.device.to_numpy(a)), as_float(hip.device.to_numpy(b)))


def as_float(values):
    values = np.asarray(values)
    return bf16_to_float32(values) if values.dtype == BFLOAT16 else values.astype(np.float32)


@pytest.mark.gpu
def test_c5_speculative_full_shape_equals_greedy(hip, tinyllama_runtime):
    """C5: 2-layer dim-512 fp16 draft proposing k = 4 for the TinyLlama-shape
    fp16 target, 5-token verification blocks, 256-token random prompt, 256
    tokens: the speculative tokens equal the target's greedy decoding token
    for token (tinyllama_speculative.py:122-123).  Greedy runs at the same
    fixed context (256 + 256 + 1 positions with the bonus block), as the
    reference's comparison does with its own context."""
    print("[gpu case] C5 speculative, full shape", flush=True)
    draft_spec = synthetic.DRAFT
    target = tinyllama_runtime
    draft = LlamaRuntime(draft_spec.config, synthetic.weights_as_tensors(
        synthetic.host_weights(draft_spec.config, draft_spec.dtype, seed=1)), compiler="hip", dtype=draft_spec.dtype)
    prompt = synthetic.prompt_ids(target.config.vocab_size, 256, seed=0).tolist()
    greedy = target.generate(prompt, 257, loop="resident")["generated_token_ids"][:256]
    for loop in ("resident", "reference"):
        result = target.generate_speculative(draft, prompt, 256, speculative_tokens=4, bonus=True, loop=loop)
        assert result["generated_tokens"] == 256
        spec = result["generated_token_ids"]
        first = next((i for i, (a, b) in enumerate(zip(spec, greedy)) if a != b), None)
        assert first is None, f"{loop}: speculative and greedy part at token {first}: {spec[first]} != {greedy[first]}"
        print(f"C5 {loop} loop: {result['warm_tokens_per_second']:.1f} tok/s, acceptance "
              f"{result['acceptance_rate']:.3f}, {result['target_verification_calls']} verification blocks", flush=True)
