"""Seeded synthetic models and prompts for the benchmark configurations.

Recipe (identical for the GPU run, the CPU baseline and the test fixtures):
* ``rng = np.random.default_rng(seed)``; walk ``required_weight_shapes`` in
  insertion order; every ``*norm.weight`` is ones and draws nothing; every
  other tensor is ``rng.normal(0, 0.02, shape)`` as float32, then cast to the
  model dtype (bf16: round to nearest even).
* With ``tie_embeddings`` the ``lm_head.weight`` entry is skipped and bound to
  the embedding tensor (Llama-3.2-1B ties them).
* Prompt ids: ``np.random.default_rng(seed + 1).integers(0, V, S, int32)``.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from .dtypes import BFLOAT16, as_dtype
from .llama import LlamaConfig, required_weight_shapes
from .tensor import Tensor


@dataclass(frozen=True)
class ModelSpec:
    name: str
    config: LlamaConfig
    dtype: np.dtype
    tie_embeddings: bool = False


def _cfg(vocab, hidden, ffn, layers, heads, kv, theta=10_000.0, max_pos=8192) -> LlamaConfig:
    return LlamaConfig(
        vocab_size=vocab, hidden_size=hidden, intermediate_size=ffn,
        num_hidden_layers=layers, num_attention_heads=heads,
        num_key_value_heads=kv, max_position_embeddings=max_pos,
        rms_norm_eps=1e-5, rope_theta=theta,
    )


TINY = ModelSpec("tiny-llama-2l-d256", _cfg(1024, 256, 688, 2, 4, 2), np.dtype(np.float32))
TINYLLAMA = ModelSpec("tinyllama-1.1b-shape", _cfg(32000, 2048, 5632, 22, 32, 4), np.dtype(np.float16))
LLAMA32_1B = ModelSpec(
    "llama-3.2-1b-shape", _cfg(128256, 2048, 8192, 16, 32, 8, theta=500_000.0),
    BFLOAT16, tie_embeddings=True,
)
DRAFT = ModelSpec("draft-2l-d512", _cfg(32000, 512, 1376, 2, 8, 4), np.dtype(np.float16))


def host_weights(
    config: LlamaConfig, dtype: object, seed: int, *, tie_embeddings: bool = False
) -> Dict[str, np.ndarray]:
    """Host arrays for every weight name (tied names share one array)."""
    rng = np.random.default_rng(seed)
    result: Dict[str, np.ndarray] = {}
    for name, shape in required_weight_shapes(config).items():
        if tie_embeddings and name == "lm_head.weight":
            continue
        if name.endswith("norm.weight"):
            result[name] = as_dtype(np.ones(shape, dtype=np.float32), dtype)
        else:
            result[name] = as_dtype(rng.normal(0.0, 0.02, shape).astype(np.float32), dtype)
    if tie_embeddings:
        result["lm_head.weight"] = result["model.embed_tokens.weight"]
    return result


def weights_as_tensors(host: Dict[str, np.ndarray]) -> Dict[str, Tensor]:
    """Wrap host arrays as leaves; tied names share one ``Tensor``."""
    by_id: Dict[int, Tensor] = {}
    result: Dict[str, Tensor] = {}
    for name, value in host.items():
        tensor = by_id.get(id(value))
        if tensor is None:
            tensor = Tensor(value, copy=False)
            by_id[id(value)] = tensor
        result[name] = tensor
    return result


def prompt_ids(vocab_size: int, length: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed + 1).integers(0, vocab_size, length, dtype=np.int32)


def weights_digest(host: Dict[str, np.ndarray], names: Optional[list] = None) -> str:
    """sha256 over names and raw bytes, to detect a drifting recipe."""
    digest = hashlib.sha256()
    for name in names or list(host):
        digest.update(name.encode())
        digest.update(np.ascontiguousarray(host[name]).view(np.uint8).tobytes())
    return digest.hexdigest()
