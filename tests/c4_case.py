"""The C4 workload (Llama-3.2-1B shape, bfloat16, tied embedding/LM head,
RoPE theta 5e5, batch 8, per-sequence KV caches of 4096 filled positions plus
room to decode) as one batched decode step; ``layers`` may be reduced for
oracle comparisons (every per-layer shape stays at its full size)."""

from __future__ import annotations

import numpy as np

from chomikgrad import Tensor, synthetic
from chomikgrad.dtypes import as_dtype
from chomikgrad.llama import LlamaBatchedDecoderStep, LlamaConfig, _rope_rotations, decode_masks

BATCH, FILLED, CONTEXT = 8, 4096, 4160


def config(layers: int) -> LlamaConfig:
    full = synthetic.LLAMA32_1B.config
    return LlamaConfig(**{**full.__dict__, "num_hidden_layers": layers})


def build(layers: int, seed: int = 0, *, float32: bool = False):
    """Returns (config, weights, leaves, cache tensors, outputs) of one
    batched decode step; sequence b decodes at position FILLED + 7 b over a
    cache of random rows (the filled prompt) with zero rows after it.  With
    ``float32`` the same bfloat16 values are widened to float32 and the step
    is built in float32 (a higher-precision reference for the same inputs)."""
    from chomikgrad.dtypes import bf16_to_float32

    spec = synthetic.LLAMA32_1B
    cfg = config(layers)
    dtype = np.dtype(np.float32) if float32 else spec.dtype
    widen = (lambda a: bf16_to_float32(a)) if float32 else (lambda a: a)
    host = synthetic.host_weights(cfg, spec.dtype, seed=seed, tie_embeddings=True)
    if float32:
        tied = host["lm_head.weight"] is host["model.embed_tokens.weight"]
        host = {k: widen(v) for k, v in host.items()}
        if tied:
            host["lm_head.weight"] = host["model.embed_tokens.weight"]
    weights = synthetic.weights_as_tensors(host)
    rng = np.random.default_rng(seed + 100)
    positions = np.array([FILLED + 7 * b for b in range(BATCH)], np.int32)
    caches = []
    for _ in range(2 * layers):
        rows = np.zeros((BATCH, cfg.num_key_value_heads, CONTEXT, cfg.head_size), np.float32)
        for b, p in enumerate(positions):
            rows[b, :, :p] = rng.normal(0.0, 0.5, (cfg.num_key_value_heads, p, cfg.head_size))
        caches.append(Tensor(widen(as_dtype(rows, spec.dtype)), copy=False))
    attention = np.concatenate([decode_masks(int(p), CONTEXT, np.float32)[0] for p in positions])
    write = np.concatenate([decode_masks(int(p), CONTEXT, np.float32)[1] for p in positions])
    rotation = np.concatenate([_rope_rotations(1, cfg.head_size, cfg.rope_theta, np.float32, offset=int(p))
                               for p in positions])
    tokens = rng.integers(0, cfg.vocab_size, (BATCH, 1)).astype(np.int32)
    cast = lambda a: widen(as_dtype(a, spec.dtype))
    leaves = [Tensor(tokens, copy=False),
              Tensor(cast(rotation.reshape(BATCH, 1, 1, 64, 64)), copy=False),
              Tensor(cast(attention.reshape(BATCH, 1, 1, CONTEXT)), copy=False),
              Tensor(cast(write.reshape(BATCH, 1, CONTEXT, 1)), copy=False),
              Tensor(positions, copy=False)]
    step = LlamaBatchedDecoderStep(cfg, weights, batch=BATCH, cache_length=CONTEXT, dtype=dtype)
    outputs = step(*leaves[:4], list(zip(caches[::2], caches[1::2])), position=leaves[4])
    return cfg, weights, leaves, caches, outputs
