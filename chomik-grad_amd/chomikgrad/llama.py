"""Llama decoder graphs written only with the six IR operations.

The node structure of every builder matches the reference's
chomikgrad/llama.py, because the portable graph fixes where a float16 or
bfloat16 computation rounds:

* ``LlamaConfig``                 -- llama.py:28-97
* ``required_weight_shapes``      -- llama.py:100-124
* ``_rope_rotations``             -- llama.py:127-152 (rotate-half as a
  row-vector rotation matrix, fp32 angles ``pos * theta^(-2i/hd)``)
* ``token_one_hot`` / ``position_selector`` -- llama.py:155-183
* ``load_safetensors``            -- llama.py:186-203
* ``LlamaForCausalLM``            -- llama.py:212-433 (prefill)
* ``LlamaDecoderStep``            -- llama.py:436-543 (one cached token)
* ``LlamaDecoderBlock``           -- llama.py:546-668 (verify a block)

``LlamaBatchedDecoderStep`` has no reference counterpart: the reference's
decode step is batch-1 only (llama.py:468-479).  It extends the same
construction to ``B`` independent sequences, each with its own cache and
position.

Optional lowering tags (``rms_norm``, ``rope``, ``sdpa``) sit on the output
node of each composite while the portable expansion stays in the graph.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Mapping, Optional, Sequence, Tuple

import numpy as np

from .dtypes import as_dtype
from .lazy import DeviceAdapter
from .tensor import Tensor


def _tag(output: Tensor, kind: str, inputs: Sequence[Tensor], argument: object) -> Tensor:
    output._node.lowering = (kind, tuple(t._node for t in inputs), argument)
    return output


@dataclass(frozen=True)
class LlamaConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    max_position_embeddings: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10_000.0
    bos_token_id: int = 1
    eos_token_id: int = 2

    @classmethod
    def from_dict(cls, config: Mapping[str, object]) -> "LlamaConfig":
        needed = (
            "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
            "num_attention_heads", "num_key_value_heads", "max_position_embeddings",
        )
        missing = [name for name in needed if name not in config]
        if missing:
            raise ValueError(f"missing Llama config fields: {', '.join(missing)}")
        result = cls(
            **{name: int(config[name]) for name in needed},
            rms_norm_eps=float(config.get("rms_norm_eps", 1e-5)),
            rope_theta=float(config.get("rope_theta", 10_000.0)),
            bos_token_id=int(config.get("bos_token_id", 1)),
            eos_token_id=int(config.get("eos_token_id", 2)),
        )
        result.validate()
        return result

    @property
    def head_size(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def query_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    def validate(self) -> None:
        sizes = (
            self.vocab_size, self.hidden_size, self.intermediate_size,
            self.num_hidden_layers, self.num_attention_heads,
            self.num_key_value_heads, self.max_position_embeddings,
        )
        if any(size <= 0 for size in sizes):
            raise ValueError("Llama dimensions must be positive")
        if self.hidden_size % self.num_attention_heads:
            raise ValueError("hidden size must be divisible by attention heads")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("attention heads must be divisible by KV heads")
        if self.head_size % 2:
            raise ValueError("RoPE requires an even attention head size")


def required_weight_shapes(config: LlamaConfig) -> Dict[str, Tuple[int, ...]]:
    """Hugging Face weight names and shapes, in the reference's order."""
    d, f = config.hidden_size, config.intermediate_size
    kv = config.num_key_value_heads * config.head_size
    shapes: Dict[str, Tuple[int, ...]] = {
        "model.embed_tokens.weight": (config.vocab_size, d),
        "model.norm.weight": (d,),
        "lm_head.weight": (config.vocab_size, d),
    }
    for layer in range(config.num_hidden_layers):
        p = f"model.layers.{layer}"
        shapes[f"{p}.input_layernorm.weight"] = (d,)
        shapes[f"{p}.post_attention_layernorm.weight"] = (d,)
        shapes[f"{p}.self_attn.q_proj.weight"] = (d, d)
        shapes[f"{p}.self_attn.k_proj.weight"] = (kv, d)
        shapes[f"{p}.self_attn.v_proj.weight"] = (kv, d)
        shapes[f"{p}.self_attn.o_proj.weight"] = (d, d)
        shapes[f"{p}.mlp.gate_proj.weight"] = (f, d)
        shapes[f"{p}.mlp.up_proj.weight"] = (f, d)
        shapes[f"{p}.mlp.down_proj.weight"] = (d, f)
    return shapes


def rope_cos_sin(
    positions: np.ndarray, head_size: int, theta: float
) -> Tuple[np.ndarray, np.ndarray]:
    """float32 cos/sin of ``position * theta^(-2i/head_size)``, i < hd/2.

    Every rotation in this package (the portable matrices below and the
    tables the ``hip`` plugin uploads for its fused RoPE) is derived from this
    one function, so both paths round the same float32 angles.
    """
    inverse = 1.0 / (theta ** (np.arange(0, head_size, 2, dtype=np.float32) / head_size))
    angles = np.asarray(positions, dtype=np.float32)[:, None] * inverse[None, :]
    return np.cos(angles), np.sin(angles)


def _rope_rotations(
    sequence_length: int, head_size: int, theta: float, dtype: object, *, offset: int = 0
) -> np.ndarray:
    """Rotation matrices ``(1, 1, S, hd, hd)``: a row vector times the matrix
    gives ``[x1*cos - x2*sin, x2*cos + x1*sin]`` (rotate-half)."""
    half = head_size // 2
    positions = np.arange(offset, offset + sequence_length, dtype=np.float32)
    cosine, sine = rope_cos_sin(positions, head_size, theta)
    matrix = np.zeros((sequence_length, head_size, head_size), dtype=np.float32)
    i = np.arange(half)
    matrix[:, i, i] = cosine
    matrix[:, i + half, i + half] = cosine
    matrix[:, i, i + half] = sine
    matrix[:, i + half, i] = -sine
    return _cast(matrix, dtype).reshape(1, 1, sequence_length, head_size, head_size)


def _cast(values: np.ndarray, dtype: object) -> np.ndarray:
    """Cast float32 host data to the model dtype (cos/sin rounded once)."""
    return as_dtype(values, dtype)


def token_one_hot(
    token_ids: Sequence[int], sequence_length: int, vocab_size: int,
    *, fill_token_id: int, dtype: object,
) -> np.ndarray:
    if len(token_ids) > sequence_length:
        raise ValueError("token sequence exceeds the fixed generation context")
    if not 0 <= fill_token_id < vocab_size:
        raise ValueError("fill token is outside the vocabulary")
    ids = np.full(sequence_length, fill_token_id, dtype=np.int64)
    ids[: len(token_ids)] = token_ids
    if np.any(ids < 0) or np.any(ids >= vocab_size):
        raise ValueError("token id is outside the vocabulary")
    encoded = np.zeros((1, sequence_length, vocab_size), dtype=np.float32)
    encoded[0, np.arange(sequence_length), ids] = 1
    return _cast(encoded, dtype)


def position_selector(position: int, sequence_length: int, *, dtype: object) -> np.ndarray:
    if not 0 <= position < sequence_length:
        raise ValueError("selected position is outside the generation context")
    selector = np.zeros((1, sequence_length), dtype=np.float32)
    selector[0, position] = 1
    return _cast(selector, dtype)


def decode_masks(position: int, cache_length: int, dtype: object) -> Tuple[np.ndarray, np.ndarray]:
    """Host masks of one decode step (generate_tinyllama.py:781-786):
    additive attention mask ``(1,1,1,C)`` with -1e4 after ``position`` and a
    one-hot write mask ``(1,1,C,1)`` at ``position``."""
    attention = np.full((1, 1, 1, cache_length), -1e4, dtype=np.float32)
    attention[..., : position + 1] = 0
    write = np.zeros((1, 1, cache_length, 1), dtype=np.float32)
    write[:, :, position, :] = 1
    return _cast(attention, dtype), _cast(write, dtype)


def block_masks(
    position: int, block_length: int, cache_length: int, dtype: object
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Host inputs of one verify block (generate_tinyllama.py:404-417):
    placement ``(B, C)``, write mask ``(1,1,C,1)`` and attention mask
    ``(1,1,B,C)``."""
    placement = np.zeros((block_length, cache_length), dtype=np.float32)
    rows = np.arange(block_length)
    placement[rows, position + rows] = 1
    write = placement.sum(axis=0).reshape(1, 1, cache_length, 1)
    attention = np.full((1, 1, block_length, cache_length), -1e4, dtype=np.float32)
    for row in range(block_length):
        attention[..., row, : position + row + 1] = 0
    return _cast(placement, dtype), _cast(write, dtype), _cast(attention, dtype)


def load_safetensors(
    path: Path, device: DeviceAdapter, *, dtype: Optional[object] = None
) -> Dict[str, Tensor]:
    """Load weights through a backend's adapter and wrap them as leaves."""
    native = (
        device.load_safetensors(path) if dtype is None
        else device.load_safetensors(path, dtype=np.dtype(dtype))
    )
    return {
        name: Tensor.from_native(
            value, backend=device.name, shape=tuple(value.shape), dtype=device.dtype(value)
        )
        for name, value in native.items()
    }


class LlamaForCausalLM:
    """Full-sequence forward (prefill) with an optional KV-cache output."""

    def __init__(
        self,
        config: LlamaConfig,
        weights: Mapping[str, Tensor],
        *,
        sequence_length: int,
        dtype: object,
        cache_length: Optional[int] = None,
    ) -> None:
        config.validate()
        if sequence_length <= 0 or sequence_length > config.max_position_embeddings:
            raise ValueError("invalid fixed generation context length")
        expected = required_weight_shapes(config)
        for name, shape in expected.items():
            if name not in weights:
                raise ValueError(f"missing model weight: {name}")
            if weights[name].shape != shape:
                raise ValueError(
                    f"weight {name} has shape {weights[name].shape}, expected {shape}"
                )
        self.config = config
        self.weights = dict(weights)
        self.sequence_length = sequence_length
        self.dtype = np.dtype(dtype)
        self.cache_length = cache_length
        self.cache_placement: Optional[Tensor] = None
        if cache_length is not None:
            if cache_length < sequence_length:
                raise ValueError("KV cache cannot be shorter than the prompt")
            placement = np.zeros((sequence_length, cache_length), dtype=np.float32)
            placement[np.arange(sequence_length), np.arange(sequence_length)] = 1
            self.cache_placement = Tensor(_cast(placement, self.dtype))
        mask = np.triu(np.full((sequence_length, sequence_length), -1e4, dtype=np.float32), k=1)
        self.causal_mask = Tensor(_cast(mask, self.dtype).reshape(1, 1, sequence_length, sequence_length))
        self.rotations = Tensor(
            _rope_rotations(sequence_length, config.head_size, config.rope_theta, self.dtype)
        )
        self.kv_repeat = Tensor.ones((1, 1, config.query_groups, 1, 1), dtype=self.dtype)

    @property
    def parameter_count(self) -> int:
        unique = {id(t._node): t for t in self.weights.values()}
        return sum(int(np.prod(t.shape)) for t in unique.values())

    # -- building blocks ----------------------------------------------------
    @staticmethod
    def _linear(inputs: Tensor, weight: Tensor) -> Tensor:
        return inputs @ weight.T

    def _rms_norm(self, inputs: Tensor, weight: Tensor) -> Tensor:
        variance = (inputs * inputs).mean(axis=-1, keepdims=True)
        output = inputs / (variance + self.config.rms_norm_eps).sqrt() * weight
        return _tag(output, "rms_norm", (inputs, weight), self.config.rms_norm_eps)

    @staticmethod
    def _silu(inputs: Tensor) -> Tensor:
        return inputs / (1 + (-inputs).exp())

    def _rotate(self, inputs: Tensor, rotation: Tensor) -> Tensor:
        b, h, t, hd = inputs.shape
        return (inputs.reshape(b, h, t, 1, hd) @ rotation).reshape(b, h, t, hd)

    def _apply_rope(self, inputs: Tensor) -> Tensor:
        output = self._rotate(inputs, self.rotations)
        return _tag(output, "rope", (inputs,), (inputs.shape[-1], self.config.rope_theta, 0))

    def _apply_rotation(self, inputs: Tensor, rotation: Tensor, position: Optional[Tensor]) -> Tensor:
        output = self._rotate(inputs, rotation)
        if position is None:
            return output
        return _tag(
            output, "rope", (inputs, position), (inputs.shape[-1], self.config.rope_theta, 0)
        )

    def _repeat_kv(self, inputs: Tensor) -> Tensor:
        b, kv, t, hd = inputs.shape
        return (inputs.reshape(b, kv, 1, t, hd) * self.kv_repeat).reshape(
            b, self.config.num_attention_heads, t, hd
        )

    def _sdpa(self, query: Tensor, key: Tensor, value: Tensor, mask: Tensor) -> Tensor:
        """Portable GQA attention tagged ``sdpa`` over the un-repeated K/V."""
        hd = self.config.head_size
        scores = (query @ self._repeat_kv(key).transpose(-2, -1)) / np.sqrt(hd) + mask
        attended = scores.softmax(axis=-1) @ self._repeat_kv(value)
        return _tag(attended, "sdpa", (query, key, value, mask), 1 / np.sqrt(hd))

    def _project_heads(self, inputs: Tensor, name: str, heads: int) -> Tensor:
        b, t, _ = inputs.shape
        return self._linear(inputs, self.weights[name]).reshape(
            b, t, heads, self.config.head_size
        ).permute(0, 2, 1, 3)

    def _attention(self, inputs: Tensor, layer: int) -> Tuple[Tensor, Tensor, Tensor]:
        c = self.config
        p = f"model.layers.{layer}.self_attn"
        b, t, _ = inputs.shape
        query = self._project_heads(inputs, f"{p}.q_proj.weight", c.num_attention_heads)
        key = self._project_heads(inputs, f"{p}.k_proj.weight", c.num_key_value_heads)
        value = self._project_heads(inputs, f"{p}.v_proj.weight", c.num_key_value_heads)
        query = self._apply_rope(query)
        key = self._apply_rope(key)
        attended = self._sdpa(query, key, value, self.causal_mask)
        merged = attended.permute(0, 2, 1, 3).reshape(b, t, c.hidden_size)
        return self._linear(merged, self.weights[f"{p}.o_proj.weight"]), key, value

    def _mlp(self, inputs: Tensor, layer: int) -> Tensor:
        p = f"model.layers.{layer}.mlp"
        gate = self._silu(self._linear(inputs, self.weights[f"{p}.gate_proj.weight"]))
        up = self._linear(inputs, self.weights[f"{p}.up_proj.weight"])
        return self._linear(gate * up, self.weights[f"{p}.down_proj.weight"])

    def _embed(self, token_matrix: Tensor) -> Tensor:
        table = self.weights["model.embed_tokens.weight"]
        if token_matrix.ndim == 2:
            return table.gather(token_matrix)
        return token_matrix @ table

    def _place(self, rows: Tensor, placement: Tensor) -> Tensor:
        """Scatter ``(1, KV, T, hd)`` rows into cache slots via a 0/1 matrix."""
        return (rows.permute(0, 1, 3, 2) @ placement).permute(0, 1, 3, 2)

    def _forward(self, token_matrix: Tensor, selector: Tensor, *, collect_cache: bool) -> Tuple[Tensor, ...]:
        c = self.config
        s = self.sequence_length
        if token_matrix.shape not in ((1, s), (1, s, c.vocab_size)):
            raise ValueError("token matrix has the wrong fixed-context shape")
        if selector.shape != (1, s):
            raise ValueError("position selector has the wrong shape")
        hidden = self._embed(token_matrix)
        caches = []
        for layer in range(c.num_hidden_layers):
            p = f"model.layers.{layer}"
            normalized = self._rms_norm(hidden, self.weights[f"{p}.input_layernorm.weight"])
            attended, key, value = self._attention(normalized, layer)
            hidden = hidden + attended
            if collect_cache:
                if self.cache_placement is None:
                    raise RuntimeError("prefill requires a configured KV cache length")
                caches.extend((self._place(key, self.cache_placement),
                               self._place(value, self.cache_placement)))
            normalized = self._rms_norm(hidden, self.weights[f"{p}.post_attention_layernorm.weight"])
            hidden = hidden + self._mlp(normalized, layer)
        hidden = self._rms_norm(hidden, self.weights["model.norm.weight"])
        selected = (selector @ hidden).reshape(1, c.hidden_size)
        logits = self._linear(selected, self.weights["lm_head.weight"])
        return (logits, *caches)

    def __call__(self, token_matrix: Tensor, selector: Tensor) -> Tensor:
        return self._forward(token_matrix, selector, collect_cache=False)[0]

    def prefill(self, token_matrix: Tensor, selector: Tensor) -> Tuple[Tensor, ...]:
        """``(logits (1, V), K0, V0, ..., K_{L-1}, V_{L-1})``."""
        return self._forward(token_matrix, selector, collect_cache=True)


class LlamaDecoderStep(LlamaForCausalLM):
    """One cached autoregressive step (batch 1)."""

    def __init__(self, config: LlamaConfig, weights: Mapping[str, Tensor], *, cache_length: int, dtype: object) -> None:
        super().__init__(config, weights, sequence_length=1, dtype=dtype)
        if cache_length <= 0 or cache_length > config.max_position_embeddings:
            raise ValueError("invalid KV cache length")
        self.cache_length = cache_length

    def _check_caches(self, caches: Sequence[Tuple[Tensor, Tensor]], batch: int = 1) -> None:
        c = self.config
        if len(caches) != c.num_hidden_layers:
            raise ValueError("decode requires one KV cache pair per layer")
        expected = (batch, c.num_key_value_heads, self.cache_length, c.head_size)
        for key, value in caches:
            if key.shape != expected or value.shape != expected:
                raise ValueError("KV cache has the wrong shape")

    def __call__(
        self,
        token_matrix: Tensor,
        rotation: Tensor,
        attention_mask: Tensor,
        write_mask: Tensor,
        caches: Sequence[Tuple[Tensor, Tensor]],
        *,
        position: Optional[Tensor] = None,
    ) -> Tuple[Tensor, ...]:
        """Returns ``(logits (1, V), K0', V0', ...)`` with functional caches."""
        c = self.config
        hd = c.head_size
        if token_matrix.shape not in ((1, 1), (1, 1, c.vocab_size)):
            raise ValueError("decode token matrix must contain exactly one token")
        if rotation.shape != (1, 1, 1, hd, hd):
            raise ValueError("decode RoPE rotation has the wrong shape")
        if attention_mask.shape != (1, 1, 1, self.cache_length):
            raise ValueError("decode attention mask has the wrong shape")
        if write_mask.shape != (1, 1, self.cache_length, 1):
            raise ValueError("decode cache write mask has the wrong shape")
        if position is not None and position.shape != ():
            raise ValueError("decode position must be a scalar")
        self._check_caches(caches)

        hidden = self._embed(token_matrix)
        updated = []
        for layer, (cached_key, cached_value) in enumerate(caches):
            p = f"model.layers.{layer}"
            a = f"{p}.self_attn"
            normalized = self._rms_norm(hidden, self.weights[f"{p}.input_layernorm.weight"])
            query = self._linear(normalized, self.weights[f"{a}.q_proj.weight"]).reshape(
                1, c.num_attention_heads, 1, hd)
            key = self._linear(normalized, self.weights[f"{a}.k_proj.weight"]).reshape(
                1, c.num_key_value_heads, 1, hd)
            value = self._linear(normalized, self.weights[f"{a}.v_proj.weight"]).reshape(
                1, c.num_key_value_heads, 1, hd)
            query = self._apply_rotation(query, rotation, position)
            key = self._apply_rotation(key, rotation, position)
            cached_key = cached_key * (1 - write_mask) + key * write_mask
            cached_value = cached_value * (1 - write_mask) + value * write_mask
            updated.append((cached_key, cached_value))
            attended = self._sdpa(query, cached_key, cached_value, attention_mask)
            merged = attended.permute(0, 2, 1, 3).reshape(1, 1, c.hidden_size)
            hidden = hidden + self._linear(merged, self.weights[f"{a}.o_proj.weight"])
            normalized = self._rms_norm(hidden, self.weights[f"{p}.post_attention_layernorm.weight"])
            hidden = hidden + self._mlp(normalized, layer)
        hidden = self._rms_norm(hidden, self.weights["model.norm.weight"])
        logits = self._linear(hidden.reshape(1, c.hidden_size), self.weights["lm_head.weight"])
        return (logits, *[t for pair in updated for t in pair])


class LlamaBatchedDecoderStep(LlamaDecoderStep):
    """``B`` independent sequences advanced by one token each.

    Inputs: tokens ``(B, 1)`` int32, rotation ``(B, 1, 1, hd, hd)``,
    attention mask ``(B, 1, 1, C)``, write mask ``(B, 1, C, 1)``, caches
    ``(B, KV, C, hd)`` per layer, optional positions ``(B,)`` int32.
    Outputs: logits ``(B, V)`` and the updated caches.
    """

    def __init__(self, config: LlamaConfig, weights: Mapping[str, Tensor], *, batch: int, cache_length: int, dtype: object) -> None:
        super().__init__(config, weights, cache_length=cache_length, dtype=dtype)
        if batch <= 0:
            raise ValueError("batch must be positive")
        self.batch = batch

    def __call__(  # type: ignore[override]
        self,
        token_matrix: Tensor,
        rotation: Tensor,
        attention_mask: Tensor,
        write_mask: Tensor,
        caches: Sequence[Tuple[Tensor, Tensor]],
        *,
        position: Optional[Tensor] = None,
    ) -> Tuple[Tensor, ...]:
        c = self.config
        b, hd, cl = self.batch, c.head_size, self.cache_length
        if token_matrix.shape != (b, 1):
            raise ValueError("batched decode tokens must have shape (batch, 1)")
        if rotation.shape != (b, 1, 1, hd, hd):
            raise ValueError("batched decode rotation has the wrong shape")
        if attention_mask.shape != (b, 1, 1, cl):
            raise ValueError("batched decode attention mask has the wrong shape")
        if write_mask.shape != (b, 1, cl, 1):
            raise ValueError("batched decode write mask has the wrong shape")
        if position is not None and position.shape != (b,):
            raise ValueError("batched decode positions must have shape (batch,)")
        self._check_caches(caches, batch=b)

        hidden = self._embed(token_matrix)
        updated = []
        for layer, (cached_key, cached_value) in enumerate(caches):
            p = f"model.layers.{layer}"
            a = f"{p}.self_attn"
            normalized = self._rms_norm(hidden, self.weights[f"{p}.input_layernorm.weight"])
            query = self._linear(normalized, self.weights[f"{a}.q_proj.weight"]).reshape(
                b, c.num_attention_heads, 1, hd)
            key = self._linear(normalized, self.weights[f"{a}.k_proj.weight"]).reshape(
                b, c.num_key_value_heads, 1, hd)
            value = self._linear(normalized, self.weights[f"{a}.v_proj.weight"]).reshape(
                b, c.num_key_value_heads, 1, hd)
            query = self._apply_rotation(query, rotation, position)
            key = self._apply_rotation(key, rotation, position)
            cached_key = cached_key * (1 - write_mask) + key * write_mask
            cached_value = cached_value * (1 - write_mask) + value * write_mask
            updated.append((cached_key, cached_value))
            attended = self._sdpa(query, cached_key, cached_value, attention_mask)
            merged = attended.permute(0, 2, 1, 3).reshape(b, 1, c.hidden_size)
            hidden = hidden + self._linear(merged, self.weights[f"{a}.o_proj.weight"])
            normalized = self._rms_norm(hidden, self.weights[f"{p}.post_attention_layernorm.weight"])
            hidden = hidden + self._mlp(normalized, layer)
        hidden = self._rms_norm(hidden, self.weights["model.norm.weight"])
        logits = self._linear(hidden.reshape(b, c.hidden_size), self.weights["lm_head.weight"])
        return (logits, *[t for pair in updated for t in pair])


class LlamaDecoderBlock(LlamaForCausalLM):
    """Verify ``block_length`` cached positions in one graph."""

    def __init__(
        self, config: LlamaConfig, weights: Mapping[str, Tensor], *,
        block_length: int, cache_length: int, dtype: object,
    ) -> None:
        super().__init__(config, weights, sequence_length=block_length, dtype=dtype)
        if cache_length < block_length or cache_length > config.max_position_embeddings:
            raise ValueError("invalid KV cache length")
        self.block_length = block_length
        self.cache_length = cache_length

    def __call__(
        self,
        token_matrix: Tensor,
        rotation: Tensor,
        attention_mask: Tensor,
        cache_placement: Tensor,
        write_mask: Tensor,
        caches: Sequence[Tuple[Tensor, Tensor]],
        *,
        position: Optional[Tensor] = None,
    ) -> Tuple[Tensor, ...]:
        """Returns ``(logits (1, B, V), K0', V0', ...)``."""
        c = self.config
        n, hd, cl = self.block_length, c.head_size, self.cache_length
        if token_matrix.shape not in ((1, n), (1, n, c.vocab_size)):
            raise ValueError("decode block has the wrong token shape")
        if rotation.shape != (1, 1, n, hd, hd):
            raise ValueError("decode block RoPE rotation has the wrong shape")
        if attention_mask.shape != (1, 1, n, cl):
            raise ValueError("decode block attention mask has the wrong shape")
        if cache_placement.shape != (n, cl):
            raise ValueError("decode block cache placement has the wrong shape")
        if write_mask.shape != (1, 1, cl, 1):
            raise ValueError("decode block write mask has the wrong shape")
        if len(caches) != c.num_hidden_layers:
            raise ValueError("decode block requires one KV cache pair per layer")
        if position is not None and position.shape != ():
            raise ValueError("decode block position must be a scalar")
        for key, value in caches:
            if key.shape != (1, c.num_key_value_heads, cl, hd) or value.shape != key.shape:
                raise ValueError("KV cache has the wrong shape")

        hidden = self._embed(token_matrix)
        updated = []
        for layer, (cached_key, cached_value) in enumerate(caches):
            p = f"model.layers.{layer}"
            a = f"{p}.self_attn"
            normalized = self._rms_norm(hidden, self.weights[f"{p}.input_layernorm.weight"])
            query = self._linear(normalized, self.weights[f"{a}.q_proj.weight"]).reshape(
                1, n, c.num_attention_heads, hd).permute(0, 2, 1, 3)
            key = self._linear(normalized, self.weights[f"{a}.k_proj.weight"]).reshape(
                1, n, c.num_key_value_heads, hd).permute(0, 2, 1, 3)
            value = self._linear(normalized, self.weights[f"{a}.v_proj.weight"]).reshape(
                1, n, c.num_key_value_heads, hd).permute(0, 2, 1, 3)
            query = self._apply_rotation(query, rotation, position)
            key = self._apply_rotation(key, rotation, position)
            cached_key = cached_key * (1 - write_mask) + self._place(key, cache_placement)
            cached_value = cached_value * (1 - write_mask) + self._place(value, cache_placement)
            updated.append((cached_key, cached_value))
            attended = self._sdpa(query, cached_key, cached_value, attention_mask)
            merged = attended.permute(0, 2, 1, 3).reshape(1, n, c.hidden_size)
            hidden = hidden + self._linear(merged, self.weights[f"{a}.o_proj.weight"])
            normalized = self._rms_norm(hidden, self.weights[f"{p}.post_attention_layernorm.weight"])
            hidden = hidden + self._mlp(normalized, layer)
        hidden = self._rms_norm(hidden, self.weights["model.norm.weight"])
        logits = self._linear(hidden, self.weights["lm_head.weight"])
        return (logits, *[t for pair in updated for t in pair])
