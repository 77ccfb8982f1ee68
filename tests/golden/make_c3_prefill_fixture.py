"""Float32-upcast oracle run of the C3 prefill (labelled as such).

Config C3: the TinyLlama-1.1B-shape model with float16 weights from seed 0
(``synthetic.TINYLLAMA``), a 2048-token prompt (``synthetic.prompt_ids``,
seed 0) and a cache of 2048 positions, prefilled in one pass
(llama.py:382-433).  The literal float16 oracle would take hours here
(NumPy's float16 matmul is a single-threaded loop), so the same weights are
upcast to float32 and this build's NumPy ``cpu`` oracle
(oracle/numpy_plugin.py) evaluates the same prefill graph in float32.

Stored (small): the last-row logits as top-32 (index, value) pairs, the
values at 1024 fixed vocabulary ids and the top-2 margin; and the K and V
cache rows of layers 0, 10 and 21 at 32 fixed positions (first and last
rows, tile edges, the middle and random rows).  About a minute and a half on
8 cores, with about 12 GB of memory.
"""

from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(REPO / "chomik-grad_amd"), str(REPO)]

import oracle  # noqa: E402,F401  registers "cpu"
from chomikgrad import synthetic  # noqa: E402
from chomikgrad.runtime import LlamaRuntime  # noqa: E402

PROMPT = 2048
SEED = 0
TOP = 32
SAMPLED = 1024
LAYERS = (0, 10, 21)


def cache_positions() -> np.ndarray:
    fixed = [0, 1, 2, 15, 16, 63, 64, 127, 128, 255, 256, 1023, 1024, 2046, 2047]
    extra = np.random.default_rng(77).choice(np.setdiff1d(np.arange(PROMPT), fixed), 32 - len(fixed),
                                             replace=False)
    return np.sort(np.concatenate([fixed, extra])).astype(np.int32)


def main() -> None:
    spec = synthetic.TINYLLAMA
    host16 = synthetic.host_weights(spec.config, spec.dtype, SEED)
    host32 = {name: value.astype(np.float32) for name, value in host16.items()}
    del host16
    runtime = LlamaRuntime(spec.config, synthetic.weights_as_tensors(host32), compiler="cpu", dtype=np.float32)
    prompt = synthetic.prompt_ids(spec.config.vocab_size, PROMPT, SEED)
    sampled = np.sort(np.random.default_rng(1234).choice(spec.config.vocab_size, SAMPLED, replace=False))
    positions = cache_positions()
    started = time.perf_counter()
    logits, caches = runtime.prefill(prompt, PROMPT)
    row = np.asarray(logits, dtype=np.float32).reshape(-1)
    order = np.argsort(-row, kind="stable")[:TOP]
    top2 = np.sort(row)[-2:]
    keys = np.stack([np.asarray(caches[2 * layer])[0][:, positions] for layer in LAYERS])
    values = np.stack([np.asarray(caches[2 * layer + 1])[0][:, positions] for layer in LAYERS])
    np.savez_compressed(
        HERE / "c3_prefill_fp32up.npz",
        prompt_length=np.array(PROMPT),
        token=np.array(int(order[0])),
        margin=np.array(top2[1] - top2[0], np.float32),
        top_index=order.astype(np.int32),
        top_value=row[order].astype(np.float32),
        sampled_index=sampled.astype(np.int32),
        sampled_value=row[sampled].astype(np.float32),
        cache_layers=np.array(LAYERS, np.int32),
        cache_positions=positions,
        keys=keys.astype(np.float32),
        values=values.astype(np.float32),
        seconds=np.array(time.perf_counter() - started),
    )
    print("token", int(order[0]), "margin", float(top2[1] - top2[0]), "seconds", time.perf_counter() - started)


if __name__ == "__main__":
    main()
