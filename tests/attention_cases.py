"""Decode-attention graphs for the planner and GPU tests: the decode step's
attention chain exactly as llama.py builds it (LlamaDecoderStep, after the
reference's llama.py:509-525) -- RoPE tagged with the position, the blended
cache write, GQA attention tagged ``sdpa`` -- over random q, k, v and caches,
for any batch, head grouping, cache length, write mask and attention mask."""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from chomikgrad import Tensor
from chomikgrad.dtypes import BFLOAT16, as_dtype
from chomikgrad.llama import _rope_rotations, _tag


@dataclass
class Case:
    name: str
    dtype: object
    B: int
    H: int
    KV: int
    C: int
    positions: Sequence[int]
    write: str = "one_hot"      # "one_hot" or "fractional"
    mask: str = "causal"        # "causal" or "per_head"
    theta: float = 10000.0
    seed: int = 0


CASES: List[Case] = [
    Case("c2-shape-fp16", np.float16, 1, 32, 4, 640, [600]),
    Case("c4-shape-bf16", BFLOAT16, 2, 32, 8, 4160, [4100, 17], theta=500000.0),
    Case("c1-shape-fp32", np.float32, 1, 4, 2, 48, [20]),
    Case("g1-fractional-per-head-fp16", np.float16, 3, 8, 8, 100, [99, 0, 50], write="fractional", mask="per_head"),
    Case("g4-short-bf16", BFLOAT16, 1, 8, 2, 37, [36]),
    Case("g2-fractional-fp32", np.float32, 2, 4, 2, 70, [3, 69], write="fractional", mask="per_head"),
    Case("g2-fractional-per-head-bf16", BFLOAT16, 2, 8, 4, 150, [149, 6], write="fractional", mask="per_head"),
]


def build(case: Case, *, positions_input: bool = True):
    """Returns (outputs [attention, K', V'], dynamic leaves, cache leaves)."""
    dtype = case.dtype
    rng = np.random.default_rng(case.seed)
    B, H, KV, C = case.B, case.H, case.KV, case.C
    G = H // KV

    def leaf(shape, scale=1.0):
        return Tensor(as_dtype((rng.normal(size=shape) * scale).astype(np.float32), dtype), copy=False)

    q, k, v = leaf((B, H, 1, 64)), leaf((B, KV, 1, 64)), leaf((B, KV, 1, 64))
    caches = [leaf((B, KV, C, 64)), leaf((B, KV, C, 64))]
    positions = np.asarray(case.positions, np.int32)
    rotation = np.concatenate([_rope_rotations(1, 64, case.theta, np.float32, offset=int(p)) for p in positions])
    rotation = Tensor(as_dtype(rotation.reshape(B, 1, 1, 64, 64), dtype), copy=False)
    position = Tensor(positions if B > 1 else positions.reshape(()), copy=False)
    write = np.zeros((B, 1, C, 1), np.float32)
    write[np.arange(B), 0, positions, 0] = 1
    if case.write == "fractional":
        write[:, 0, ::7, 0] = 0.25
        write[np.arange(B), 0, positions, 0] = 1
    if case.mask == "causal":
        attention = np.full((B, 1, 1, C), -1e4, np.float32)
        for b, p in enumerate(positions):
            attention[b, ..., : p + 1] = 0
    else:
        attention = (rng.normal(size=(B, H, 1, C)) * 2).astype(np.float32)
        attention[..., ::5] = -1e4
    write_t = Tensor(as_dtype(write, dtype), copy=False)
    attention_t = Tensor(as_dtype(attention, dtype), copy=False)

    def rope(x):
        b, h, t, d = x.shape
        out = (x.reshape(b, h, t, 1, d) @ rotation).reshape(b, h, t, d)
        return _tag(out, "rope", (x, position), (d, case.theta, 0)) if positions_input else out

    ones = Tensor.ones((1, 1, G, 1, 1), dtype=dtype)

    def repeat(x):
        b, kv, t, d = x.shape
        return (x.reshape(b, kv, 1, t, d) * ones).reshape(b, kv * G, t, d)

    qr, kr = rope(q), rope(k)
    K = caches[0] * (1 - write_t) + kr * write_t
    V = caches[1] * (1 - write_t) + v * write_t
    scores = (qr @ repeat(K).transpose(-2, -1)) / np.sqrt(64) + attention_t
    attended = _tag(scores.softmax(axis=-1) @ repeat(V), "sdpa", (qr, K, V, attention_t), 1 / np.sqrt(64))
    dynamic = [q, k, v, rotation, position, write_t, attention_t, *caches]
    return [attended, K, V], dynamic, caches


def tolerance(case: Case):
    if np.dtype(case.dtype) == np.float32:
        return dict(rtol=1e-4, atol=1e-5)
    if np.dtype(case.dtype) == np.float16:
        return dict(rtol=1e-2, atol=3e-3)
    return dict(rtol=3e-2, atol=2e-2)
