"""Float32-upcast oracle run of the C2 headline workload (labelled as such).

Config C2: the TinyLlama-1.1B-shape model with float16 weights from seed 0
(``synthetic.TINYLLAMA``), the 512-token prompt of seed 0, a fixed context of
640 positions (512 + 128 new tokens, as the benchmark runs it).  The literal
float16 oracle would take about 40 minutes for the 512-token prefill alone
(NumPy's float16 matmul is a single-threaded loop), so the same weights are
upcast to float32 and this build's NumPy ``cpu`` oracle
(oracle/numpy_plugin.py) runs the reference-protocol loop in float32: the
prefill, then 32 greedy decode steps at positions 512..543
(generate_tinyllama.py:712-857).  A float16 evaluation differs from this one
by float16 rounding only, so the GPU test holds it to the north-star float16
tolerance and requires equal greedy tokens wherever the top-2 margin is
clear of that noise.

Stored (small): the tokens, each step's top-2 margin, the top-32 (index,
value) pairs of each logits row and the logits at 1024 fixed vocabulary ids.
Takes about a minute on 8 cores.
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

PROMPT = 512
CONTEXT = 640
STEPS = 32
SEED = 0
TOP = 32
SAMPLED = 1024


def main() -> None:
    spec = synthetic.TINYLLAMA
    host16 = synthetic.host_weights(spec.config, spec.dtype, SEED)
    host32 = {name: value.astype(np.float32) for name, value in host16.items()}
    runtime = LlamaRuntime(spec.config, synthetic.weights_as_tensors(host32), compiler="cpu", dtype=np.float32)
    prompt = synthetic.prompt_ids(spec.config.vocab_size, PROMPT, SEED)
    sampled = np.sort(np.random.default_rng(1234).choice(spec.config.vocab_size, SAMPLED, replace=False))
    started = time.perf_counter()
    logits, caches = runtime.prefill(prompt, CONTEXT)
    rows, tokens = [], []
    for step in range(STEPS + 1):
        row = np.asarray(logits, dtype=np.float32).reshape(-1)
        rows.append(row)
        token = int(np.argmax(row))
        tokens.append(token)
        if step == STEPS:
            break
        logits, caches = runtime._decode_step(token, PROMPT + step, CONTEXT, caches)
        print(f"step {step} token {token} {time.perf_counter() - started:.1f}s", flush=True)
    rows = np.stack(rows)
    order = np.argsort(-rows, axis=1, kind="stable")[:, :TOP]
    top2 = np.sort(rows, axis=1)[:, -2:]
    np.savez_compressed(
        HERE / "c2_ctx512_fp32up.npz",
        prompt=prompt,
        context=np.array(CONTEXT),
        tokens=np.asarray(tokens[:STEPS + 1], dtype=np.int64),
        margins=(top2[:, 1] - top2[:, 0]).astype(np.float32),
        top_index=order.astype(np.int32),
        top_value=np.take_along_axis(rows, order, axis=1).astype(np.float32),
        sampled_index=sampled.astype(np.int32),
        sampled_value=rows[:, sampled].astype(np.float32),
        weights_digest=np.array(synthetic.weights_digest(host16, ["model.embed_tokens.weight",
                                                                  "model.layers.0.self_attn.q_proj.weight",
                                                                  "lm_head.weight"])),
        seconds=np.array(time.perf_counter() - started),
    )
    print("tokens", tokens)
    print("margins", np.round(top2[:, 1] - top2[:, 0], 4).tolist())
    print("seconds", time.perf_counter() - started)


if __name__ == "__main__":
    main()
