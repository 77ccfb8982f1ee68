"""Write golden vectors by running the REFERENCE's own ``cpu`` plugin.

Runs only in the build container, where /root/reference exists; never on the
GPU box.  The reference package cannot be imported as ``chomikgrad`` under
Python 3.10 (its CUDA/OpenCL plugin files use 3.12 f-string syntax and
``__init__`` imports them), so this script registers an empty package named
``refchomik`` whose path is the reference's ``chomikgrad`` directory and
imports only ``lazy``, ``tensor``, ``llama`` and ``generation`` from it.

What it pins (nothing else can): the bit-level result of the reference's
composed Llama graphs as executed by its NumpyCompiler
(chomikgrad/lazy.py:551-636), following its greedy driver
(examples/generate_tinyllama.py:712-857) with the EOS stop disabled.

* ``c1_greedy.npz``: config C1 (2 layers, D 256, 4/2 heads, FFN 688,
  V 1024, fp32, seed 0), 16-token prompt, 32 greedy tokens, all logits.
* ``fp16_step.npz``: one TinyLlama-shape fp16 layer (D 2048, 32/4 heads,
  FFN 5632) with a 1024-token vocabulary: 8-token prefill then 4 decode
  steps, all logits (float16).

Inputs are regenerated from the seed with the recipe in
``chomikgrad/synthetic.py``; the fixture stores a digest of the weights so
a drifting recipe is detected.
"""

from __future__ import annotations

import importlib
import sys
import types
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO / "chomik-grad_amd"))

from chomikgrad import synthetic  # noqa: E402  (the input recipe)

REFERENCE = Path("/root/reference/chomikgrad")


def load_reference():
    package = types.ModuleType("refchomik")
    package.__path__ = [str(REFERENCE)]
    sys.modules["refchomik"] = package
    lazy = importlib.import_module("refchomik.lazy")
    tensor = importlib.import_module("refchomik.tensor")
    llama = importlib.import_module("refchomik.llama")
    return lazy, tensor, llama


def greedy(ref, spec_config, dtype, host, prompt, new_tokens):
    """The reference driver's greedy loop on its cpu plugin (no EOS stop)."""
    lazy, tensor_mod, llama = ref
    Tensor = tensor_mod.Tensor
    config = llama.LlamaConfig(**{
        field: getattr(spec_config, field) for field in (
            "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
            "num_attention_heads", "num_key_value_heads", "max_position_embeddings",
            "rms_norm_eps", "rope_theta", "bos_token_id", "eos_token_id")
    })
    weights = {name: Tensor(value) for name, value in host.items()}
    context = len(prompt) + new_tokens
    model = llama.LlamaForCausalLM(config, weights, sequence_length=len(prompt),
                                   dtype=dtype, cache_length=context)
    tokens = list(int(t) for t in prompt)
    inputs = np.asarray(tokens, dtype=np.int32).reshape(1, -1)
    selector = llama.position_selector(len(prompt) - 1, len(prompt), dtype=dtype)
    outputs = tensor_mod.compile_graph(*model.prefill(Tensor(inputs, copy=False),
                                                      Tensor(selector, copy=False)),
                                       compiler="cpu").run(synchronize=True)
    logits = [np.asarray(outputs[0]).copy()]
    token = int(np.asarray(outputs[0]).argmax())
    tokens.append(token)
    caches = list(outputs[1:])
    decoder = llama.LlamaDecoderStep(config, weights, cache_length=context, dtype=dtype)
    program = None
    nodes = None
    for _ in range(1, new_tokens):
        position = len(tokens) - 1
        step_inputs = np.asarray([[token]], dtype=np.int32)
        rotation = llama._rope_rotations(1, config.head_size, config.rope_theta, dtype,
                                         offset=position)
        attention = np.full((1, 1, 1, context), -1e4, dtype=dtype)
        attention[..., : position + 1] = 0
        write = np.zeros((1, 1, context, 1), dtype=dtype)
        write[:, :, position, :] = 1
        position_value = np.asarray(position, dtype=np.int32)
        if program is None:
            leaves = [Tensor(step_inputs, copy=False), Tensor(rotation, copy=False),
                      Tensor(attention, copy=False), Tensor(write, copy=False),
                      Tensor(position_value, copy=False)]
            cache_tensors = [Tensor(np.asarray(c), copy=False) for c in caches]
            graph = decoder(*leaves[:4], list(zip(cache_tensors[::2], cache_tensors[1::2])),
                            position=leaves[4])
            program = tensor_mod.compile_graph(*graph, compiler="cpu",
                                               dynamic_inputs=leaves + cache_tensors)
            nodes = [t._node for t in leaves + cache_tensors]
            outputs = program.run(synchronize=True)
        else:
            values = [step_inputs, rotation, attention, write, position_value, *caches]
            outputs = program.run(dict(zip(nodes, values)), synchronize=True)
        logits.append(np.asarray(outputs[0]).copy())
        token = int(np.asarray(outputs[0]).argmax())
        tokens.append(token)
        caches = list(outputs[1:])
    return np.asarray(tokens[len(prompt):], dtype=np.int64), np.concatenate(logits, axis=0)


def main() -> None:
    ref = load_reference()

    spec = synthetic.TINY
    host = synthetic.host_weights(spec.config, spec.dtype, seed=0)
    prompt = synthetic.prompt_ids(spec.config.vocab_size, 16, seed=0)
    tokens, logits = greedy(ref, spec.config, spec.dtype, host, prompt, 32)
    np.savez_compressed(
        HERE / "c1_greedy.npz", prompt=prompt, tokens=tokens, logits=logits,
        weights_digest=np.array(synthetic.weights_digest(host)),
    )
    print("c1 tokens", tokens.tolist())

    config = synthetic._cfg(1024, 2048, 5632, 1, 32, 4)
    host16 = synthetic.host_weights(config, np.float16, seed=3)
    prompt16 = synthetic.prompt_ids(config.vocab_size, 8, seed=3)
    tokens16, logits16 = greedy(ref, config, np.dtype(np.float16), host16, prompt16, 5)
    np.savez_compressed(
        HERE / "fp16_step.npz", prompt=prompt16, tokens=tokens16, logits=logits16,
        weights_digest=np.array(synthetic.weights_digest(host16)),
    )
    print("fp16 tokens", tokens16.tolist())


if __name__ == "__main__":
    main()
