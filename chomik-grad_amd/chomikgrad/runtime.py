"""Generation driver: the counterpart of the reference's ``TinyLlamaRuntime``
(examples/generate_tinyllama.py:165-263) for in-memory weights.

``LlamaRuntime.generate`` follows ``_generate_loaded``
(generate_tinyllama.py:678-887): context = prompt + max_new_tokens; the first
token comes from the prefill program; then ``max_new_tokens - 1`` decode
steps at ``position = len(tokens) - 1``; prefill programs are cached by
``(prompt_len, context)`` and decode programs by ``context``.  Two loops:

* ``loop="reference"`` -- the reference's per-step protocol on any compiler:
  host-built token, rotation, masks and position are uploaded with
  ``device.array`` every step, caches are functional, and every token is
  copied to the host by ``device.argmax`` (sample_native_token,
  generate_tinyllama.py:146-162).
* ``loop="resident"`` (``hip`` only, greedy) -- only the token, position and
  KV caches feed each step, and all of them stay on the device: the caches
  are donated and updated in place, and one queued ``greedy_advance`` writes
  the next token, position and masks.  The host waits once, at the end.

The EOS stop (generate_tinyllama.py:770) is optional; fixed-length runs
disable it.
"""

from __future__ import annotations

import statistics
import time
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .generation import verify_greedy_block_with_bonus
from .lazy import get_compiler
from .llama import (
    LlamaConfig,
    LlamaDecoderBlock,
    LlamaDecoderStep,
    LlamaForCausalLM,
    _rope_rotations,
    block_masks,
    decode_masks,
    position_selector,
)
from .tensor import Tensor, compile_graph, no_grad


def sample_token(logits: np.ndarray, *, temperature: float, top_k: int, rng: np.random.Generator) -> int:
    """Host sampling (generate_tinyllama.py:124-143): greedy at temperature
    0, else softmax over the top-k logits scaled by 1/temperature."""
    values = np.asarray(logits, dtype=np.float64).reshape(-1)
    if temperature == 0:
        return int(values.argmax())
    values = values / temperature
    if 0 < top_k < values.size:
        keep = np.argpartition(values, -top_k)[-top_k:]
        filtered = np.full_like(values, -np.inf)
        filtered[keep] = values[keep]
        values = filtered
    values -= values.max()
    probabilities = np.exp(values)
    probabilities /= probabilities.sum()
    return int(rng.choice(values.size, p=probabilities))


def _host_float(values: np.ndarray) -> np.ndarray:
    from .dtypes import BFLOAT16, bf16_to_float32
    values = np.asarray(values)
    return bf16_to_float32(values) if values.dtype == BFLOAT16 else values.astype(np.float32)


class LlamaRuntime:
    def __init__(self, config: LlamaConfig, weights: Dict[str, Tensor], *,
                 compiler: str = "hip", dtype: Optional[object] = None) -> None:
        self.config = config
        self.weights = weights
        self.compiler_name = compiler
        self.compiler = get_compiler(compiler)
        self.device = self.compiler.device
        self.dtype = np.dtype(dtype if dtype is not None else getattr(self.device, "inference_dtype", np.float32))
        self._prefill_programs: Dict[Tuple[int, int], Tuple[Any, Any]] = {}
        self._decoder_programs: Dict[Tuple[int, bool], Tuple[Any, List[Any]]] = {}
        self._block_programs: Dict[Tuple[int, int], Tuple[Any, List[Any]]] = {}

    # -- prefill ----------------------------------------------------------------
    def prefill(self, prompt: Sequence[int], context: int):
        """Run (and cache) the prefill program: returns (logits, caches)."""
        key = (len(prompt), context)
        inputs = np.asarray(prompt, dtype=np.int32).reshape(1, -1)
        cached = self._prefill_programs.get(key)
        if cached is None:
            model = LlamaForCausalLM(self.config, self.weights, sequence_length=len(prompt),
                                     dtype=self.dtype, cache_length=context)
            token_tensor = Tensor(inputs, copy=False)
            selector = Tensor(position_selector(len(prompt) - 1, len(prompt), dtype=self.dtype), copy=False)
            outputs = model.prefill(token_tensor, selector)
            program = compile_graph(*outputs, compiler=self.compiler_name, dynamic_inputs=(token_tensor,))
            self._prefill_programs[key] = (program, token_tensor._node)
            bindings = None
        else:
            program, node = cached
            bindings = {node: self.device.array(inputs)}
        native = program.run(bindings, synchronize=False)
        return native[0], list(native[1:])

    # -- decode program -------------------------------------------------------------
    def _decoder(self, context: int, position: int, caches: List[Any], *, donate: bool):
        key = (context, donate)
        cached = self._decoder_programs.get(key)
        if cached is not None:
            return cached
        c = self.config
        rotation = _rope_rotations(1, c.head_size, c.rope_theta, self.dtype, offset=position)
        attention, write = decode_masks(position, context, self.dtype)
        leaves = [
            Tensor(np.zeros((1, 1), dtype=np.int32), copy=False),
            Tensor(rotation, copy=False),
            Tensor(attention, copy=False),
            Tensor(write, copy=False),
            Tensor(np.asarray(position, dtype=np.int32), copy=False),
        ]
        cache_tensors = [
            Tensor.from_native(value, backend=self.device.name, shape=tuple(value.shape), dtype=self.dtype)
            for value in caches
        ]
        decoder = LlamaDecoderStep(c, self.weights, cache_length=context, dtype=self.dtype)
        outputs = decoder(*leaves[:4], list(zip(cache_tensors[::2], cache_tensors[1::2])), position=leaves[4])
        dynamic = leaves + cache_tensors
        kwargs = {}
        if donate:
            kwargs["donate"] = [t._node for t in cache_tensors]
        program = self.compiler.compile([o._node for o in outputs], [t._node for t in dynamic], **kwargs)
        entry = (program, [t._node for t in dynamic])
        self._decoder_programs[key] = entry
        return entry

    # -- verification block (speculative decoding) -------------------------------------
    def _verifier(self, block: int, context: int, position: int, caches: List[Any]):
        """Compile (once per (block, context)) the target's verification block:
        ``block`` tokens at ``position`` against the caches, returning their
        logits (1, block, V) and the caches with the block written
        (generate_tinyllama.py:396-488, LlamaDecoderBlock).  Caches are
        donated: the block updates them in place."""
        key = (block, context)
        cached = self._block_programs.get(key)
        if cached is not None:
            return cached
        c = self.config
        placement, write, attention = block_masks(position, block, context, self.dtype)
        leaves = [
            Tensor(np.zeros((1, block), dtype=np.int32), copy=False),
            Tensor(_rope_rotations(block, c.head_size, c.rope_theta, self.dtype, offset=position), copy=False),
            Tensor(attention, copy=False),
            Tensor(placement, copy=False),
            Tensor(write, copy=False),
            Tensor(np.asarray(position, dtype=np.int32), copy=False),
        ]
        cache_tensors = [
            Tensor.from_native(value, backend=self.device.name, shape=tuple(value.shape), dtype=self.dtype)
            for value in caches
        ]
        decoder = LlamaDecoderBlock(c, self.weights, block_length=block, cache_length=context, dtype=self.dtype)
        outputs = decoder(*leaves[:5], list(zip(cache_tensors[::2], cache_tensors[1::2])), position=leaves[5])
        dynamic = leaves + cache_tensors
        kwargs = {"donate": [t._node for t in cache_tensors]} if self.compiler_name == "hip" else {}
        program = self.compiler.compile([o._node for o in outputs], [t._node for t in dynamic], **kwargs)
        entry = (program, [t._node for t in dynamic])
        self._block_programs[key] = entry
        return entry

    def _decode_step(self, token: int, position: int, context: int, caches: List[Any]):
        """One decode step with host-built rotation and masks (the reference's
        _run_decoder_step, generate_tinyllama.py:309-393): returns (logits,
        caches)."""
        c = self.config
        donate = self.compiler_name == "hip"
        program, nodes = self._decoder(context, position, caches, donate=donate)
        attention, write = decode_masks(position, context, self.dtype)
        values = [
            self.device.array(np.asarray([[token]], dtype=np.int32)),
            self.device.array(_rope_rotations(1, c.head_size, c.rope_theta, self.dtype, offset=position)),
            self.device.array(attention),
            self.device.array(write),
            self.device.array(np.asarray(position, dtype=np.int32)),
            *caches,
        ]
        native = program.run(dict(zip(nodes, values)), synchronize=False)
        return native[0], list(native[1:])

    def _verify_block(self, inputs: Sequence[int], position: int, context: int, caches: List[Any]):
        """Run the verification block over ``inputs`` at ``position``: returns
        the target's greedy prediction after each input and the caches."""
        logits, caches = self._verify_block_logits(inputs, position, context, caches)
        predictions = np.asarray(self.device.argmax_last_axis(logits)).reshape(-1)
        return [int(t) for t in predictions], caches

    def _verify_block_logits(self, inputs: Sequence[int], position: int, context: int, caches: List[Any]):
        """The verification block's logits (1, len(inputs), V) and caches."""
        c = self.config
        block = len(inputs)
        program, nodes = self._verifier(block, context, position, caches)
        placement, write, attention = block_masks(position, block, context, self.dtype)
        values = [
            self.device.array(np.asarray([inputs], dtype=np.int32)),
            self.device.array(_rope_rotations(block, c.head_size, c.rope_theta, self.dtype, offset=position)),
            self.device.array(attention),
            self.device.array(placement),
            self.device.array(write),
            self.device.array(np.asarray(position, dtype=np.int32)),
            *caches,
        ]
        native = program.run(dict(zip(nodes, values)), synchronize=False)
        return native[0], list(native[1:])

    def generate_speculative(
        self,
        draft: "LlamaRuntime",
        prompt: Sequence[int],
        max_new_tokens: int,
        *,
        speculative_tokens: int = 4,
        draft_prompt: Optional[Sequence[int]] = None,
        bonus: bool = False,
        stop_at_eos: bool = False,
        loop: Optional[str] = None,
    ) -> Dict[str, object]:
        """Greedy speculative decoding with ``draft`` proposing for this
        (target) runtime -- the reference's _generate_speculative_loaded
        (generate_tinyllama.py:491-622):

        * the first token comes from the target's prefill; the draft prefills
          its own prompt (``draft_prompt``, default the same ids);
        * each round the draft proposes up to ``speculative_tokens`` greedy
          tokens, one decode step each, starting from the last emitted token;
        * the target verifies them in one block and the longest agreeing
          prefix plus the target's own next token is emitted
          (verify_greedy_candidates, generation.py:15-28).

        ``bonus=False`` is the reference's block ``[last, d1 .. d_{k-1}]``
        (k predictions, no extra token when all k agree).  ``bonus=True``
        verifies ``[last, d1 .. dk]`` (k + 1 predictions): when all k agree
        the target's prediction after ``dk`` is emitted as well, and the
        draft, which never consumed ``dk``, catches up with one extra step
        before its next proposal.  Either way the emitted sequence equals the
        target's own greedy decoding.

        ``loop="reference"`` drives every step from the host, as the
        reference does; ``loop="resident"`` (the default on the hip plugin)
        keeps a round on the device and synchronises once per round."""
        from .generation import verify_greedy_candidates

        if max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be positive")
        if speculative_tokens <= 0:
            raise ValueError("speculative_tokens must be positive")
        if not len(prompt):
            raise ValueError("the prompt produced no tokens")
        draft_prompt = list(prompt) if draft_prompt is None else list(draft_prompt)
        context = len(prompt) + max_new_tokens + (1 if bonus else 0)
        draft_context = len(draft_prompt) + max_new_tokens + 1
        for runtime, length in ((self, context), (draft, draft_context)):
            if length > runtime.config.max_position_embeddings:
                raise ValueError(f"prompt plus output is {length} tokens, model limit is "
                                 f"{runtime.config.max_position_embeddings}")
        if loop is None:
            loop = "resident" if self.compiler_name == "hip" and draft.compiler_name == "hip" else "reference"
        if loop == "resident":
            return self._speculative_resident(draft, prompt, draft_prompt, max_new_tokens, speculative_tokens,
                                              bonus, stop_at_eos, context, draft_context)
        if loop != "reference":
            raise ValueError(f"unknown loop {loop!r}")
        eos = self.config.eos_token_id
        started = time.perf_counter()
        with no_grad():
            logits, target_caches = self.prefill(prompt, context)
            token = self.device.argmax(logits)
            first_token_seconds = time.perf_counter() - started
            _, draft_caches = draft.prefill(draft_prompt, draft_context)
            generated = [token]
            tokens = list(prompt) + [token]
            decode_started = time.perf_counter()
            accepted = proposed = verifications = draft_calls = 0
            lagging: Optional[int] = None  # a token the draft has not consumed yet
            while len(generated) < max_new_tokens and not (stop_at_eos and token == eos):
                limit = min(speculative_tokens, max_new_tokens - len(generated))
                draft_position = len(draft_prompt) + len(generated) - 1
                if lagging is not None:  # consume dk before proposing from the bonus token
                    _, draft_caches = draft._decode_step(lagging, draft_position - 1, draft_context, draft_caches)
                    draft_calls += 1
                    lagging = None
                proposal: List[int] = []
                draft_token = token
                for _ in range(limit):
                    draft_logits, draft_caches = draft._decode_step(draft_token, draft_position, draft_context,
                                                                    draft_caches)
                    draft_token = draft.device.argmax(draft_logits)
                    proposal.append(draft_token)
                    draft_calls += 1
                    draft_position += 1
                    if stop_at_eos and draft_token == eos:
                        break
                block = [token, *proposal] if bonus else [token, *proposal[:-1]]
                predictions, target_caches = self._verify_block(block, len(tokens) - 1, context, target_caches)
                if bonus:
                    decision = verify_greedy_block_with_bonus(proposal, predictions)
                    if decision.accepted_draft_tokens == len(proposal):
                        lagging = proposal[-1]
                else:
                    decision = verify_greedy_candidates(proposal, predictions)
                emitted = list(decision.emitted_tokens)[: max_new_tokens - len(generated)]
                if stop_at_eos and eos in emitted:
                    emitted = emitted[: emitted.index(eos) + 1]
                tokens.extend(emitted)
                generated.extend(emitted)
                token = emitted[-1]
                accepted += decision.accepted_draft_tokens
                proposed += len(proposal)
                verifications += 1
            self.device.synchronize()
        decode_seconds = time.perf_counter() - decode_started
        decode_tokens = len(generated) - 1
        return {
            "loop": "speculative" + ("-bonus" if bonus else ""),
            "generated_token_ids": generated,
            "prompt_tokens": len(prompt),
            "generated_tokens": len(generated),
            "first_token_seconds": first_token_seconds,
            "decode_seconds": decode_seconds,
            "warm_tokens_per_second": decode_tokens / decode_seconds if decode_tokens else None,
            "wall_generation_seconds": time.perf_counter() - started,
            "fixed_context_tokens": context,
            "speculative_tokens": speculative_tokens,
            "accepted_draft_tokens": accepted,
            "proposed_draft_tokens": proposed,
            "acceptance_rate": accepted / proposed if proposed else 0.0,
            "target_verification_calls": verifications,
            "draft_decode_calls": draft_calls,
            "kv_cache": True,
        }

    def _speculative_resident(self, draft, prompt, draft_prompt, max_new_tokens, speculative_tokens, bonus,
                              stop_at_eos, context, draft_context):
        """One host synchronisation per round: the draft's proposals feed its
        next step on the device (greedy_advance writes each token into the
        draft's input and into the verification block's token row), the
        block's per-row greedy predictions stay on the device, and the host
        reads back only the block's tokens and predictions to apply the
        acceptance rule.  Masks and positions of a round follow from the
        round's start position, which the host knows, and are uploaded
        without waiting.  Same tokens as the reference loop."""
        from .generation import verify_greedy_candidates

        device = draft.device
        eos = self.config.eos_token_id
        k = speculative_tokens
        width = k + 1 if bonus else k  # block rows: [last, d1 .. dk] or [last, d1 .. d_{k-1}]
        started = time.perf_counter()
        with no_grad():
            logits, target_caches = self.prefill(prompt, context)
            token = device.argmax(logits)
            first_token_seconds = time.perf_counter() - started
            _, draft_caches = draft.prefill(draft_prompt, draft_context)
            generated = [token]
            decode_started = time.perf_counter()
            # device state of the draft loop and of the block
            proposals = device.empty((1, k + 1), np.int32)  # [last, d1 .. dk]
            block_tokens = device.view(proposals, 0, (1, width))
            draft_token = device.empty((1, 1), np.int32)
            draft_pos = device.empty((), np.int32)
            d_attention_host, d_write_host = decode_masks(0, draft_context, draft.dtype)
            d_attention = device.array(d_attention_host)
            d_write = device.array(d_write_host)
            d_program, d_nodes = draft._decoder(draft_context, len(draft_prompt), draft_caches, donate=True)
            d_logits = device.empty(d_program._planned.output_nodes[0].shape, draft.dtype)
            d_rotation = device.array(_rope_rotations(1, draft.config.head_size, draft.config.rope_theta,
                                                      draft.dtype, offset=0))
            d_bindings = dict(zip(d_nodes, [draft_token, d_rotation, d_attention, d_write, draft_pos,
                                            *draft_caches]))
            placement_host, write_host, attention_host = block_masks(len(prompt), width, context, self.dtype)
            b_attention = device.array(attention_host)
            b_placement = device.array(placement_host)
            b_write = device.array(write_host)
            b_pos = device.empty((), np.int32)
            b_program, b_nodes = self._verifier(width, context, len(prompt), target_caches)
            b_logits = device.empty(b_program._planned.output_nodes[0].shape, self.dtype)
            b_rotation = device.array(_rope_rotations(width, self.config.head_size, self.config.rope_theta,
                                                      self.dtype, offset=0))
            b_bindings = dict(zip(b_nodes, [block_tokens, b_rotation, b_attention, b_placement, b_write, b_pos,
                                            *target_caches]))
            predictions = device.empty((width,), np.int32)
            accepted = proposed = verifications = draft_calls = 0
            lagging: Optional[int] = None
            while len(generated) < max_new_tokens and not (stop_at_eos and token == eos):
                limit = min(k, max_new_tokens - len(generated))
                draft_position = len(draft_prompt) + len(generated) - 1
                if lagging is not None:  # the draft consumes dk (its logits are not needed)
                    device.upload(draft_token, np.array([[lagging]], np.int32))
                    device.upload(draft_pos, np.asarray(draft_position - 1, np.int32))
                    attention_host, write_host = decode_masks(draft_position - 1, draft_context, draft.dtype)
                    device.upload(d_attention, attention_host)
                    device.upload(d_write, write_host)
                    d_program.run(d_bindings, out=[d_logits])
                    draft_calls += 1
                    lagging = None
                device.upload(draft_token, np.array([[token]], np.int32))
                device.upload(proposals, np.array([[token] + [0] * k], np.int32))
                device.upload(draft_pos, np.asarray(draft_position, np.int32))
                attention_host, write_host = decode_masks(draft_position, draft_context, draft.dtype)
                device.upload(d_attention, attention_host)
                device.upload(d_write, write_host)
                for step in range(1, limit + 1):
                    d_program.run(d_bindings, out=[d_logits])
                    device.greedy_advance(d_logits, draft_token, history=proposals, step=step, position=draft_pos,
                                          attention_mask=d_attention, write_mask=d_write,
                                          cache_length=draft_context)
                draft_calls += limit
                position = len(prompt) + len(generated) - 1
                rows = limit + 1 if bonus else limit
                if rows != width:  # a short last round: its own block program
                    block = device.to_numpy(proposals).reshape(-1)[:rows].tolist()
                    preds, target_caches = self._verify_block(block, position, context, target_caches)
                    proposal = device.to_numpy(proposals).reshape(-1)[1:limit + 1].tolist()
                else:
                    placement_host, write_host, attention_host = block_masks(position, width, context, self.dtype)
                    device.upload(b_attention, attention_host)
                    device.upload(b_placement, placement_host)
                    device.upload(b_write, write_host)
                    device.upload(b_pos, np.asarray(position, np.int32))
                    b_program.run(b_bindings, out=[b_logits])
                    device.greedy_advance(b_logits, predictions)
                    preds = device.to_numpy(predictions).tolist()  # the round's one wait
                    proposal = device.to_numpy(proposals).reshape(-1)[1:limit + 1].tolist()
                if stop_at_eos and eos in proposal:
                    proposal = proposal[: proposal.index(eos) + 1]
                    preds = preds[: len(proposal) + (1 if bonus else 0)]
                if bonus:
                    decision = verify_greedy_block_with_bonus(proposal, preds)
                    if decision.accepted_draft_tokens == len(proposal):
                        lagging = proposal[-1]
                else:
                    decision = verify_greedy_candidates(proposal, preds)
                emitted = list(decision.emitted_tokens)[: max_new_tokens - len(generated)]
                if stop_at_eos and eos in emitted:
                    emitted = emitted[: emitted.index(eos) + 1]
                generated.extend(emitted)
                token = emitted[-1]
                accepted += decision.accepted_draft_tokens
                proposed += len(proposal)
                verifications += 1
            device.synchronize()
        decode_seconds = time.perf_counter() - decode_started
        decode_tokens = len(generated) - 1
        return {
            "loop": "speculative-resident" + ("-bonus" if bonus else ""),
            "generated_token_ids": generated,
            "prompt_tokens": len(prompt),
            "generated_tokens": len(generated),
            "first_token_seconds": first_token_seconds,
            "decode_seconds": decode_seconds,
            "warm_tokens_per_second": decode_tokens / decode_seconds if decode_tokens else None,
            "wall_generation_seconds": time.perf_counter() - started,
            "fixed_context_tokens": context,
            "speculative_tokens": speculative_tokens,
            "accepted_draft_tokens": accepted,
            "proposed_draft_tokens": proposed,
            "acceptance_rate": accepted / proposed if proposed else 0.0,
            "target_verification_calls": verifications,
            "draft_decode_calls": draft_calls,
            "kv_cache": True,
        }

    # -- generation ------------------------------------------------------------------
    def generate(
        self,
        prompt: Sequence[int],
        max_new_tokens: int,
        *,
        temperature: float = 0.0,
        top_k: int = 50,
        seed: int = 0,
        stop_at_eos: bool = False,
        loop: Optional[str] = None,
    ) -> Dict[str, object]:
        if max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be positive")
        if not len(prompt):
            raise ValueError("the prompt produced no tokens")
        context = len(prompt) + max_new_tokens
        if context > self.config.max_position_embeddings:
            raise ValueError(f"prompt plus output is {context} tokens, model limit is "
                             f"{self.config.max_position_embeddings}")
        if loop is None:
            loop = "resident" if (self.compiler_name == "hip" and temperature == 0) else "reference"
        if loop == "resident":
            if temperature != 0:
                raise ValueError("the resident loop is greedy only")
            return self._generate_resident(prompt, max_new_tokens, context, stop_at_eos)
        return self._generate_reference(prompt, max_new_tokens, context, temperature, top_k, seed, stop_at_eos)

    def _generate_reference(self, prompt, max_new_tokens, context, temperature, top_k, seed, stop_at_eos):
        rng = np.random.default_rng(seed)
        device = self.device
        tokens = [int(t) for t in prompt]
        generated: List[int] = []
        step_seconds: List[float] = []
        started = time.perf_counter()
        with no_grad():
            step_started = time.perf_counter()
            logits, caches = self.prefill(tokens, context)
            token = self._sample(logits, temperature, top_k, rng)
            step_seconds.append(time.perf_counter() - step_started)
            tokens.append(token)
            generated.append(token)
            for _ in range(1, max_new_tokens):
                if stop_at_eos and token == self.config.eos_token_id:
                    break
                position = len(tokens) - 1
                c = self.config
                rotation = _rope_rotations(1, c.head_size, c.rope_theta, self.dtype, offset=position)
                attention, write = decode_masks(position, context, self.dtype)
                step_started = time.perf_counter()
                program, nodes = self._decoder(context, position, caches, donate=False)
                values = [
                    device.array(np.asarray([[token]], dtype=np.int32)),
                    device.array(rotation),
                    device.array(attention),
                    device.array(write),
                    device.array(np.asarray(position, dtype=np.int32)),
                    *caches,
                ]
                native = program.run(dict(zip(nodes, values)), synchronize=False)
                token = self._sample(native[0], temperature, top_k, rng)
                step_seconds.append(time.perf_counter() - step_started)
                tokens.append(token)
                generated.append(token)
                caches = list(native[1:])
        warm = step_seconds[1:]
        return {
            "loop": "reference",
            "generated_token_ids": generated,
            "prompt_tokens": len(prompt),
            "generated_tokens": len(generated),
            "first_token_seconds": step_seconds[0],
            "warm_token_median_seconds": statistics.median(warm) if warm else None,
            "warm_tokens_per_second": 1 / statistics.median(warm) if warm else None,
            "total_generation_seconds": sum(step_seconds),
            "wall_generation_seconds": time.perf_counter() - started,
            "fixed_context_tokens": context,
            "kv_cache": True,
        }

    def _sample(self, logits, temperature, top_k, rng) -> int:
        if temperature == 0:
            return self.device.argmax(logits)
        return sample_token(_host_float(self.device.to_numpy(logits)), temperature=temperature,
                            top_k=top_k, rng=rng)

    def _generate_resident(self, prompt, max_new_tokens, context, stop_at_eos):
        device = self.device
        started = time.perf_counter()
        history = device.empty((max_new_tokens,), np.int32)
        token = device.empty((1, 1), np.int32)
        with no_grad():
            first_started = time.perf_counter()
            logits, caches = self.prefill(prompt, context)
            device.greedy_advance(logits, token, history=history, step=0)
            position_value = len(prompt)
            attention_host, write_host = decode_masks(position_value, context, self.dtype)
            position = device.array(np.asarray(position_value, dtype=np.int32))
            attention = device.array(attention_host)
            write = device.array(write_host)
            device.synchronize()
            first_token_seconds = time.perf_counter() - first_started
            decode_started = time.perf_counter()
            if max_new_tokens > 1:
                program, nodes = self._decoder(context, position_value, caches, donate=True)
                placeholder_rotation = device.array(_rope_rotations(
                    1, self.config.head_size, self.config.rope_theta, self.dtype, offset=position_value))
                bindings = dict(zip(nodes, [token, placeholder_rotation, attention, write, position, *caches]))
                logits_out = device.empty(program._planned.output_nodes[0].shape, self.dtype)
                outs = [logits_out]
                for step in range(1, max_new_tokens):
                    program.run(bindings, out=outs)
                    device.greedy_advance(logits_out, token, history=history, step=step,
                                          position=position, attention_mask=attention,
                                          write_mask=write, cache_length=context)
            device.synchronize()
            decode_seconds = time.perf_counter() - decode_started
        generated = [int(t) for t in device.to_numpy(history)]
        if stop_at_eos and self.config.eos_token_id in generated:
            generated = generated[: generated.index(self.config.eos_token_id) + 1]
        decode_tokens = max_new_tokens - 1
        return {
            "loop": "resident",
            "generated_token_ids": generated,
            "prompt_tokens": len(prompt),
            "generated_tokens": len(generated),
            "first_token_seconds": first_token_seconds,
            "decode_seconds": decode_seconds,
            "warm_token_median_seconds": decode_seconds / decode_tokens if decode_tokens else None,
            "warm_tokens_per_second": decode_tokens / decode_seconds if decode_tokens else None,
            "wall_generation_seconds": time.perf_counter() - started,
            "fixed_context_tokens": context,
            "kv_cache": True,
        }
