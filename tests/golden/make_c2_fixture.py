"""Literal float16 oracle run on the TinyLlama-1.1B-shape model (config C2).

Runs this build's NumPy ``cpu`` oracle (oracle/numpy_plugin.py, the
restatement of the reference's NumpyCompiler) through the reference-protocol
greedy loop: a 32-token prompt, 32 greedy tokens, context 64.  Takes about
five minutes on 8 cores (fp16 np.matmul is NumPy's single-threaded loop), so
the result is committed as ``c2_fp16_greedy.npz`` and the GPU tests compare
against it.  Stores the tokens, the logits of every step and each step's
top-2 margin (how close a greedy choice was to a tie).
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

PROMPT = 32
NEW = 32
SEED = 0


class LogitRecorder:
    """Wraps the oracle device to keep every logits row passed to argmax."""

    def __init__(self, device):
        self.device = device
        self.rows = []
        self.name = device.name

    def __getattr__(self, name):
        return getattr(self.device, name)

    def argmax(self, value):
        self.rows.append(np.asarray(value, dtype=np.float16).reshape(-1).copy())
        return self.device.argmax(value)


def main() -> None:
    spec = synthetic.TINYLLAMA
    host = synthetic.host_weights(spec.config, spec.dtype, SEED)
    weights = synthetic.weights_as_tensors(host)
    prompt = synthetic.prompt_ids(spec.config.vocab_size, PROMPT, SEED)
    runtime = LlamaRuntime(spec.config, weights, compiler="cpu", dtype=spec.dtype)
    recorder = LogitRecorder(runtime.device)
    runtime.device = recorder
    started = time.perf_counter()
    result = runtime.generate(prompt, NEW, loop="reference")
    logits = np.stack(recorder.rows)
    top2 = np.sort(logits.astype(np.float32), axis=1)[:, -2:]
    np.savez_compressed(
        HERE / "c2_fp16_greedy.npz",
        prompt=prompt,
        tokens=np.asarray(result["generated_token_ids"], dtype=np.int64),
        logits=logits,
        margins=top2[:, 1] - top2[:, 0],
        weights_digest=np.array(synthetic.weights_digest(host, ["model.embed_tokens.weight",
                                                                 "model.layers.0.self_attn.q_proj.weight",
                                                                 "lm_head.weight"])),
        seconds=np.array(time.perf_counter() - started),
    )
    print("tokens", result["generated_token_ids"])
    print("min margin", float((top2[:, 1] - top2[:, 0]).min()), "seconds", time.perf_counter() - started)


if __name__ == "__main__":
    main()
