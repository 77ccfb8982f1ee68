"""Benchmark: TinyLlama-1.1B-shape fp16 batch-1 decode at context 512 (C2)
through the ``hip`` plugin on one MI355X.

A step is one greedy decode token.  The model is random-init (seeded,
N(0, 0.02), norms = 1), the prompt is 512 uniform random ids.  The program:
prefill of the prompt (timed separately), then ``--warmup`` untimed decode
steps, then exactly ``--steps`` timed decode steps bracketed by device
synchronisation.  Decoding uses the device-resident greedy loop (the KV
caches are donated and updated in place; token, position and masks advance
on the device; no host round trip per token).

Further fields: ``prefill_c3`` (the 2048-token C3 prefill with MFMA
utilisation and a per-kernel breakdown), ``c4_batched_decode`` (C4, 8 bf16
sequences over 4096 filled cache rows, device-resident loop) and
``c5_speculative`` (C5, draft + 5-token verification blocks) -- reported
alongside, not the headline metric.

Besides the JSON line's ``value`` (decode tok/s), ``roofline`` describes the
dominant kernel (the largest share of decode time per token) from HIP-event
timings of the real decode plan's launches, with the HBM traffic per launch
measured by FETCH_SIZE/WRITE_SIZE counter runs (profiles/decode_c2_traffic.json,
when it lists that kernel), and ``cpu_baseline`` times the NumPy oracle (the
reference's cpu plugin algorithm) on a bounded sample of the same workload on
this host.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "chomik-grad_amd"), str(ROOT)]

METRIC = "decode tok/s + % HBM roofline, TinyLlama-1.1B-shape fp16 bs=1 ctx512"
HBM_PEAK_GBPS = 8000.0
PROMPT = 512


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def kernel_label(step) -> str:
    """Kernel kind, its fusions and (for GEMVs) the weight shape N x K."""
    from chomikgrad._planner import K_GEMV, KIND_NAMES

    if step.kind != K_GEMV:
        return KIND_NAMES[step.kind]
    tags = []
    if step.attrs["prologue"]:
        tags.append("rms_norm")
    if step.attrs["silu"]:
        tags.append("silu_mul")
    if any(s["res"] is not None for s in step.attrs["segments"]):
        tags.append("residual")
    rows = sum(seg["w"].shape[0] for seg in step.attrs["segments"])
    shape = f" {rows}x{step.attrs['K']}"
    return ("gemv[" + "+".join(tags) + "]" if tags else "gemv") + shape


def algorithmic_bytes(step) -> int:
    """Bytes a kernel must move at minimum: every operand read once, every
    result written once (KV writes in place touch one row per head)."""
    from chomikgrad._planner import K_DECODE_ATTN, K_GATHER, K_GEMV, K_KV_WRITE

    if step.kind == K_GATHER:
        # the gathered rows (read once, written once) and the indices
        table, ids = step.ins[0], step.ins[1]
        out = step.outs[0]
        return 2 * out.size * out.itemsize + ids.size * ids.itemsize
    if step.kind == K_GEMV:
        total = sum(pv.size * pv.itemsize for pv in step.reads())
        return total + sum(pv.size * pv.itemsize for pv in {id(o.storage): o for o in step.outs}.values())
    if step.kind == K_DECODE_ATTN:
        # q, k, v, the position, one RoPE table row, both caches and both
        # masks read once; the output and (in place) one written row per KV
        # head and cache -- the combine scratch and tickets are not operands
        q, k, v, position, table, cache_k, cache_v, w, mask, _tickets, _partials = step.ins
        reads = sum(pv.size * pv.itemsize for pv in (q, k, v, position, cache_k, cache_v, w, mask))
        reads += table.shape[1] * table.itemsize
        out = step.outs[0]
        rows = cache_k.shape[0] * cache_k.shape[1] * cache_k.shape[3] * cache_k.itemsize
        written = 2 * rows if step.attrs.get("in_place") else 2 * cache_k.size * cache_k.itemsize
        return reads + out.size * out.itemsize + written
    if step.kind == K_KV_WRITE and step.attrs.get("in_place"):
        cache, x, w = step.ins
        row = cache.shape[0] * cache.shape[1] * cache.shape[3] * cache.itemsize
        return w.size * w.itemsize + x.size * x.itemsize + row
    total = sum(pv.size * pv.itemsize for pv in step.reads())
    return total + sum(pv.size * pv.itemsize for pv in step.outs)


def weights_bytes(config, itemsize: int) -> int:
    from chomikgrad.llama import required_weight_shapes

    shapes = required_weight_shapes(config)
    total = 0
    for name, shape in shapes.items():
        if name == "model.embed_tokens.weight":
            total += shape[1] * itemsize  # one embedding row per token
        else:
            total += int(np.prod(shape)) * itemsize
    return total


MFMA_PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 matrix peak


def prefill_flops(config, tokens: int) -> float:
    """Algorithmic FLOPs of one causal prefill: every linear over all rows,
    q.k and p.v over the causal triangle, the lm_head for the selected row."""
    from chomikgrad.llama import required_weight_shapes

    shapes = required_weight_shapes(config)
    linear = sum(int(np.prod(shape)) for name, shape in shapes.items()
                 if name.endswith("proj.weight"))
    attention = (4 * config.num_attention_heads * config.head_size * tokens * (tokens + 1) // 2
                 * config.num_hidden_layers)
    lm_head = 2 * config.hidden_size * config.vocab_size
    return 2.0 * tokens * linear + attention + lm_head


def step_flops(step) -> int:
    """Algorithmic FLOPs of a prefill matrix kernel (0 for the others):
    2 M N K for a GEMM; q.k and p.v over the visited keys for attention
    (the causal triangle when the mask was proved causal)."""
    from chomikgrad._planner import K_GEMM, K_SDPA

    if step.kind == K_GEMM:  # the SiLU pair multiplies by gate and up weights
        pair = 2 if step.attrs.get("up") is not None else 1
        return 2 * pair * step.attrs["rows"] * step.attrs["N"] * step.attrs["K"]
    if step.kind == K_SDPA:
        b, h, t, hd = step.ins[0].shape
        c = step.ins[1].shape[2]
        keys = t * (t + 1) // 2 if step.attrs.get("causal") is not None else t * c
        return 4 * b * h * hd * keys
    return 0


def plan_label(step) -> str:
    """Kernel kind plus, for GEMMs, M x N x K."""
    from chomikgrad._planner import K_GEMM, KIND_NAMES

    if step.kind == K_GEMM:
        epilogue = "+silu_pair" if step.attrs.get("up") is not None else (
            "+residual" if step.attrs.get("res") is not None else "")
        return f"gemm{epilogue} {step.attrs['rows']}x{step.attrs['N']}x{step.attrs['K']}"
    return kernel_label(step)


def plan_breakdown(program, lib, *, rounds: int, flops=None) -> dict:
    """Average duration of each kernel group of a plan: every instance of a
    label launched round-robin ``rounds`` times between one HIP event pair
    on the library stream (chip_plan_time_repeat)."""
    steps = program._planned.steps
    groups = {}
    for index, step in enumerate(steps):
        groups.setdefault(plan_label(step), []).append(index)
    out = {}
    for label, indices in groups.items():
        ids = (ctypes.c_int64 * len(indices))(*indices)
        ms = ctypes.c_float(0.0)
        lib.call("chip_plan_time_repeat", program._plan, ids, ctypes.c_int64(len(indices)),
                 ctypes.c_int64(rounds), ctypes.byref(ms))
        entry = {"launches": len(indices), "avg_us": round(1e3 * ms.value, 2),
                 "total_ms": round(ms.value * len(indices), 3)}
        if flops is not None:
            f = statistics.mean(flops(steps[i]) for i in indices)
            if f:
                entry["tflops"] = round(f / (ms.value * 1e-3) / 1e12, 1)
        out[label] = entry
    return out


def prefill_measurement(runtime, config, device, lib, tokens: int, runs: int) -> dict:
    """C3: one prompt of ``tokens`` ids through the prefill program (compiled
    and warmed first), timed with HIP events on the library stream."""
    from chomikgrad import synthetic

    prompt = synthetic.prompt_ids(config.vocab_size, tokens, seed=0)
    runtime.prefill(prompt, tokens)
    device.synchronize()
    start, stop = ctypes.c_void_p(), ctypes.c_void_p()
    lib.call("chip_event_create", ctypes.byref(start))
    lib.call("chip_event_create", ctypes.byref(stop))
    samples = []
    for _ in range(runs):
        lib.call("chip_event_record", start)
        runtime.prefill(prompt, tokens)
        lib.call("chip_event_record", stop)
        device.synchronize()
        ms = ctypes.c_float(0.0)
        lib.call("chip_event_elapsed_ms", start, stop, ctypes.byref(ms))
        samples.append(ms.value)
    lib.call("chip_event_destroy", start)
    lib.call("chip_event_destroy", stop)
    best = min(samples)
    flops = prefill_flops(config, tokens)
    tflops = flops / (best * 1e-3) / 1e12
    program = runtime._prefill_programs[(tokens, tokens)][0]
    breakdown = plan_breakdown(program, lib, rounds=2, flops=step_flops)
    return {
        "workload": f"C3: TinyLlama-1.1B-shape fp16 causal prefill of {tokens} tokens",
        "tokens": tokens, "ms": round(best, 3), "ms_runs": [round(v, 3) for v in samples],
        "tok_per_s": round(tokens / (best * 1e-3), 1),
        "algorithmic_tflop": round(flops / 1e12, 4), "achieved_tflops": round(tflops, 1),
        "peak_tflops": MFMA_PEAK_FP16_TFLOPS, "mfma_utilisation": round(tflops / MFMA_PEAK_FP16_TFLOPS, 4),
        "kernel_breakdown": breakdown,
    }


def c4_measurement(device, lib, steps: int, warmup: int) -> dict:
    """C4: Llama-3.2-1B-shape bf16 (tied embedding/LM head, RoPE theta 5e5),
    8 sequences decoding greedily together over per-sequence caches whose
    first 4096 rows are filled (synthetic rows, the same block for every
    layer) -- the device-resident batched loop, ``steps`` timed steps."""
    from chomikgrad import Tensor, synthetic
    from chomikgrad.dtypes import as_dtype
    from chomikgrad.llama import LlamaBatchedDecoderStep, _rope_rotations, decode_masks

    spec = synthetic.LLAMA32_1B
    cfg, dtype = spec.config, spec.dtype
    batch, filled = 8, 4096
    context = filled + 1 + warmup + steps
    started = time.perf_counter()
    weights = synthetic.weights_as_tensors(synthetic.host_weights(cfg, dtype, seed=0, tie_embeddings=True))
    rng = np.random.default_rng(7)
    block = np.zeros((batch, cfg.num_key_value_heads, context, cfg.head_size), np.float32)
    block[:, :, :filled] = rng.standard_normal((batch, cfg.num_key_value_heads, filled, cfg.head_size),
                                               dtype=np.float32) * 0.5
    block = as_dtype(block, dtype)
    caches = [device.array(block) for _ in range(2 * cfg.num_hidden_layers)]
    log(f"C4 weights and caches ready in {time.perf_counter() - started:.1f} s")
    positions = np.full(batch, filled, np.int32)
    attention = np.concatenate([decode_masks(filled, context, np.float32)[0]] * batch).reshape(batch, 1, 1, context)
    write = np.concatenate([decode_masks(filled, context, np.float32)[1]] * batch).reshape(batch, 1, context, 1)
    rotation = np.concatenate([_rope_rotations(1, 64, cfg.rope_theta, np.float32, offset=filled)] * batch)
    leaves = [Tensor(np.zeros((batch, 1), np.int32), copy=False),
              Tensor(as_dtype(rotation.reshape(batch, 1, 1, 64, 64), dtype), copy=False),
              Tensor(as_dtype(attention, dtype), copy=False), Tensor(as_dtype(write, dtype), copy=False),
              Tensor(positions, copy=False)]
    cache_tensors = [Tensor.from_native(c, backend=device.name, shape=tuple(c.shape), dtype=dtype) for c in caches]
    step = LlamaBatchedDecoderStep(cfg, weights, batch=batch, cache_length=context, dtype=dtype)
    outputs = step(*leaves[:4], list(zip(cache_tensors[::2], cache_tensors[1::2])), position=leaves[4])
    from chomikgrad import get_compiler
    hip = get_compiler("hip")
    program = hip.compile([o._node for o in outputs], [t._node for t in leaves + cache_tensors],
                          donate=[t._node for t in cache_tensors])
    if leaves[1]._node in program.inputs:
        raise RuntimeError("the C4 program does not lower RoPE")
    tokens = device.array(np.random.default_rng(8).integers(0, cfg.vocab_size, (batch, 1)).astype(np.int32))
    position = device.array(positions)
    attention_d = device.array(as_dtype(attention, dtype))
    write_d = device.array(as_dtype(write, dtype))
    bindings = dict(zip([t._node for t in leaves + cache_tensors],
                        [tokens, device.array(as_dtype(rotation.reshape(batch, 1, 1, 64, 64), dtype)),
                         attention_d, write_d, position, *caches]))
    logits = device.empty((batch, cfg.vocab_size), dtype)

    def run(count):
        for _ in range(count):
            program.run(bindings, out=[logits])
            device.greedy_advance(logits, tokens, position=position, attention_mask=attention_d,
                                  write_mask=write_d, cache_length=context)

    run(warmup)
    device.synchronize()
    start, stop = ctypes.c_void_p(), ctypes.c_void_p()
    lib.call("chip_event_create", ctypes.byref(start))
    lib.call("chip_event_create", ctypes.byref(stop))
    lib.call("chip_event_record", start)
    run(steps)
    lib.call("chip_event_record", stop)
    device.synchronize()
    ms = ctypes.c_float(0.0)
    lib.call("chip_event_elapsed_ms", start, stop, ctypes.byref(ms))
    lib.call("chip_event_destroy", start)
    lib.call("chip_event_destroy", stop)
    seconds = ms.value * 1e-3
    first = filled + warmup
    kv_per_position = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_size * 2
    weight_bytes = weights_bytes(cfg, 2) + (batch - 1) * cfg.hidden_size * 2  # one embedding row per sequence
    kv_bytes = batch * kv_per_position * float(np.mean(np.arange(first, first + steps) + 2))  # read p + 1, write 1
    per_step = weight_bytes + kv_bytes
    return {
        "workload": "C4: Llama-3.2-1B-shape bf16, batch 8 greedy decode over 4096 filled cache positions",
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms.value / steps, 4),
        "tok_per_s": round(batch * steps / seconds, 1),
        "bytes_per_step": int(per_step), "achieved_gbps": round(per_step * steps / seconds / 1e9, 1),
        "roofline_frac": round(per_step * steps / seconds / 1e9 / HBM_PEAK_GBPS, 4),
        "program_kernels": program.kernel_count + 1,
        "kernel_breakdown": plan_breakdown(program, lib, rounds=3),
    }


def c5_measurement(target, tokens: int, lib=None) -> dict:
    """C5: the 2-layer dim-512 fp16 draft (seed 1) proposing k = 4 greedy
    tokens per round for the C2 target, verified in 5-token blocks; 256-token
    random prompt.  Timed on the second (warm) run."""
    from chomikgrad import synthetic
    from chomikgrad.runtime import LlamaRuntime

    spec = synthetic.DRAFT
    draft = LlamaRuntime(spec.config, synthetic.weights_as_tensors(synthetic.host_weights(spec.config, spec.dtype, seed=1)),
                         compiler="hip", dtype=spec.dtype)
    prompt = synthetic.prompt_ids(target.config.vocab_size, 256, seed=0).tolist()
    target.generate_speculative(draft, prompt, tokens, speculative_tokens=4, bonus=True)
    result = target.generate_speculative(draft, prompt, tokens, speculative_tokens=4, bonus=True)
    block = {}
    if lib is not None:
        # the 5-row verification block: each kernel group's average duration
        programs = [entry[0] for key, entry in target._block_programs.items() if key[0] == 5]
        if programs:
            block = plan_breakdown(programs[0], lib, rounds=10)
    return {
        "workload": "C5: greedy speculative decoding, 2-layer dim-512 draft (k = 4) for the C2 target, "
                    "5-token verification blocks, 256-token prompt",
        "verify_block_kernels": block,
        "verify_block_kernel_ms": round(sum(v["total_ms"] for v in block.values()), 3) if block else None,
        "generated_tokens": result["generated_tokens"],
        "tok_per_s": round(result["warm_tokens_per_second"], 1),
        "acceptance_rate": round(result["acceptance_rate"], 4),
        "verification_blocks": result["target_verification_calls"],
        "draft_steps": result["draft_decode_calls"],
        "note": "independent random-init draft and target: acceptance is near 0, so each round emits the target's "
                "own token after k draft steps",
    }


def cpu_baseline(config, weights, dtype, context: int, first_position: int, steps: int) -> dict:
    """Oracle decode steps on the host: the reference's NumPy cpu-plugin
    algorithm, float16, with zero-filled caches of the real context length.
    fp16 np.matmul is NumPy's single-threaded loop, so one core is used."""
    import oracle  # noqa: F401  (the checker, timed as the CPU baseline)
    from chomikgrad import Tensor, get_compiler
    from chomikgrad.llama import LlamaDecoderStep, _rope_rotations, decode_masks

    compiler = get_compiler("cpu")
    kv = (1, config.num_key_value_heads, context, config.head_size)
    caches = [np.zeros(kv, dtype=dtype) for _ in range(2 * config.num_hidden_layers)]
    decoder = LlamaDecoderStep(config, weights, cache_length=context, dtype=dtype)
    seconds = []
    token = 1
    for step in range(steps):
        position = first_position + step
        attention, write = decode_masks(position, context, dtype)
        leaves = [Tensor(np.array([[token]], np.int32), copy=False),
                  Tensor(_rope_rotations(1, config.head_size, config.rope_theta, dtype, offset=position), copy=False),
                  Tensor(attention, copy=False), Tensor(write, copy=False)]
        cache_tensors = [Tensor(c, copy=False) for c in caches]
        outputs = decoder(*leaves, list(zip(cache_tensors[::2], cache_tensors[1::2])))
        started = time.perf_counter()
        result = compiler.compile([o._node for o in outputs]).run()
        token = int(np.asarray(result[0]).argmax())
        seconds.append(time.perf_counter() - started)
        caches = [np.asarray(c) for c in result[1:]]
    per_token = statistics.mean(seconds)
    return {
        "value": round(1.0 / per_token, 4),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{steps} fp16 decode steps of the C2 model at positions {first_position}.."
                   f"{first_position + steps - 1}, context {context}, zero-filled caches "
                   f"({per_token:.2f} s/token; host has {len(os.sched_getaffinity(0))} cores, "
                   "fp16 NumPy matmul uses one)"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=115)
    parser.add_argument("--warmup", type=int, default=8)
    parser.add_argument("--timing-runs", type=int, default=4, help="spare context rows for the kernel timing")
    parser.add_argument("--timing-rounds", type=int, default=10,
                        help="round-robin passes over each kernel's per-layer instances")
    parser.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                        help="only copy a MIB-sized device buffer three times (counter calibration) and exit")
    parser.add_argument("--cpu-steps", type=int, default=3, help="oracle decode steps for the CPU baseline")
    parser.add_argument("--prefill-tokens", type=int, default=2048, help="C3 prefill length (0 skips it)")
    parser.add_argument("--prefill-runs", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--c4-steps", type=int, default=64, help="C4 batched decode steps (0 skips it)")
    parser.add_argument("--c5-tokens", type=int, default=256, help="C5 speculative tokens (0 skips it)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs every kernel on a single MI355X and has no "
              f"collective path (--gpus {args.gpus} requested)", file=sys.stderr)
        return 2
    if args.steps < 1:
        raise SystemExit("--steps must be positive")

    from chomikgrad import get_compiler, synthetic
    from chomikgrad.llama import _rope_rotations, decode_masks
    from chomikgrad.runtime import LlamaRuntime

    spec = synthetic.TINYLLAMA
    config, dtype = spec.config, spec.dtype
    hip = get_compiler("hip")
    device = hip.device
    log(f"device {device.info}")
    if args.copy_probe:
        # A plain device-to-device copy of known size: the reference point
        # for scaling FETCH_SIZE / WRITE_SIZE counters to bytes.
        nbytes = args.copy_probe << 20
        source = device.zeros((nbytes // 2,), np.float16)
        for _ in range(3):
            device.copy(source)
        device.synchronize()
        print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}), flush=True)
        return 0
    started = time.perf_counter()
    host = synthetic.host_weights(config, dtype, seed=0)
    weights = synthetic.weights_as_tensors(host)
    log(f"weights generated in {time.perf_counter() - started:.1f} s")
    runtime = LlamaRuntime(config, weights, compiler="hip", dtype=dtype)
    prompt = synthetic.prompt_ids(config.vocab_size, PROMPT, seed=0)
    context = PROMPT + 1 + args.warmup + args.steps + args.timing_runs

    lib = hip.lib
    # Prefill (compile + one warm run, then one timed run: HIP events on the
    # library stream, and the host's wall clock, which also holds the cache
    # allocation and the uploads).
    runtime.prefill(prompt, context)
    device.synchronize()
    log("prefill compiled")
    start_event, stop_event = ctypes.c_void_p(), ctypes.c_void_p()
    lib.call("chip_event_create", ctypes.byref(start_event))
    lib.call("chip_event_create", ctypes.byref(stop_event))
    t0 = time.perf_counter()
    lib.call("chip_event_record", start_event)
    logits, caches = runtime.prefill(prompt, context)
    lib.call("chip_event_record", stop_event)
    device.synchronize()
    prefill_wall_ms = (time.perf_counter() - t0) * 1e3
    prefill_event_ms = ctypes.c_float(0.0)
    lib.call("chip_event_elapsed_ms", start_event, stop_event, ctypes.byref(prefill_event_ms))
    lib.call("chip_event_destroy", start_event)
    lib.call("chip_event_destroy", stop_event)
    prefill_ms = prefill_event_ms.value
    log(f"prefill {PROMPT} tokens: {prefill_ms:.2f} ms on the stream ({prefill_wall_ms:.1f} ms host wall)")

    history = device.empty((1 + args.warmup + args.steps + args.timing_runs,), np.int32)
    token = device.empty((1, 1), np.int32)
    device.greedy_advance(logits, token, history=history, step=0)
    attention_host, write_host = decode_masks(PROMPT, context, dtype)
    position = device.array(np.asarray(PROMPT, dtype=np.int32))
    attention = device.array(attention_host)
    write = device.array(write_host)
    program, nodes = runtime._decoder(context, PROMPT, caches, donate=True)
    rotation = device.array(_rope_rotations(1, config.head_size, config.rope_theta, dtype, offset=PROMPT))
    bindings = dict(zip(nodes, [token, rotation, attention, write, position, *caches]))
    if nodes[1] in program.inputs:
        raise RuntimeError("the decode program does not lower RoPE; the resident loop needs it")
    logits_out = device.empty((1, config.vocab_size), dtype)
    log(f"decode plan: {program.kernel_count} kernels per token")

    step_index = 1

    def decode(count: int) -> None:
        nonlocal step_index
        for _ in range(count):
            program.run(bindings, out=[logits_out])
            device.greedy_advance(logits_out, token, history=history, step=step_index, position=position,
                                  attention_mask=attention, write_mask=write, cache_length=context)
            step_index += 1

    decode(args.warmup)
    device.synchronize()
    start_event, stop_event = ctypes.c_void_p(), ctypes.c_void_p()
    lib.call("chip_event_create", ctypes.byref(start_event))
    lib.call("chip_event_create", ctypes.byref(stop_event))
    device.synchronize()
    wall0 = time.perf_counter()
    lib.call("chip_event_record", start_event)
    decode(args.steps)
    lib.call("chip_event_record", stop_event)
    device.synchronize()
    wall = time.perf_counter() - wall0
    gpu_ms = ctypes.c_float(0.0)
    lib.call("chip_event_elapsed_ms", start_event, stop_event, ctypes.byref(gpu_ms))
    first_timed_position = PROMPT + args.warmup
    tokens = device.to_numpy(history).tolist()
    log(f"timed {args.steps} steps: wall {wall * 1e3:.2f} ms, events {gpu_ms.value:.2f} ms")

    # Per-kernel durations of the same decode plan: every step of one kind
    # and shape (its per-layer instances, round-robin so no cache holds the
    # repeats) launched back to back between one HIP event pair on the
    # library stream.  The caches are donated (updated in place), so repeats
    # of the attention step rewrite the same rows with the same values.
    steps = program._planned.steps
    groups = {}
    for index, step in enumerate(steps):
        groups.setdefault(kernel_label(step), []).append(index)
    breakdown = {}
    for label, indices in groups.items():
        ids = (ctypes.c_int64 * len(indices))(*indices)
        ms = ctypes.c_float(0.0)
        lib.call("chip_plan_time_repeat", program._plan, ids, ctypes.c_int64(len(indices)),
                 ctypes.c_int64(args.timing_rounds), ctypes.byref(ms))
        per_launch_bytes = statistics.mean(algorithmic_bytes(steps[i]) for i in indices)
        breakdown[label] = {
            "launches_per_token": len(indices),
            "avg_us": round(1e3 * ms.value, 3),
            "us_per_token": round(1e3 * ms.value * len(indices), 2),
            "bytes_per_launch": int(per_launch_bytes),
            "gbps": round(per_launch_bytes / (ms.value * 1e-3) / 1e9, 1),
        }
    device.synchronize()
    dominant = max(breakdown, key=lambda k: breakdown[k]["us_per_token"])
    traffic = None
    traffic_file = ROOT / "profiles" / "decode_c2_traffic.json"
    if traffic_file.exists():
        measured = json.loads(traffic_file.read_text()).get("kernels", {}).get(dominant)
        if measured:
            traffic = measured["hbm_bytes_per_launch"]
    dom_bytes = breakdown[dominant]["bytes_per_launch"]
    dom_us = breakdown[dominant]["avg_us"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9

    decode_tps = args.steps / wall
    positions = np.arange(first_timed_position, first_timed_position + args.steps)
    kv_bytes = 2 * config.num_hidden_layers * config.num_key_value_heads * config.head_size * 2
    bytes_per_token = float(np.mean(weights_bytes(config, 2) + kv_bytes * (positions + 1) + kv_bytes))
    step_gbps = bytes_per_token * decode_tps / 1e9

    prefill_c3 = None
    if args.prefill_tokens:
        log(f"C3 prefill of {args.prefill_tokens} tokens")
        prefill_c3 = prefill_measurement(runtime, config, device, lib, args.prefill_tokens, args.prefill_runs)
        log(f"C3 prefill: {prefill_c3['ms']} ms, {prefill_c3['achieved_tflops']} TFLOP/s")

    c5 = None
    if args.c5_tokens:
        log(f"C5 speculative decoding of {args.c5_tokens} tokens")
        c5 = c5_measurement(runtime, args.c5_tokens, lib)
        log(f"C5: {c5['tok_per_s']} tok/s, acceptance {c5['acceptance_rate']}")
    c4 = None
    if args.c4_steps:
        log(f"C4 batched bf16 decode, {args.c4_steps} steps")
        c4 = c4_measurement(device, lib, args.c4_steps, 4)
        log(f"C4: {c4['tok_per_s']} tok/s, roofline {c4['roofline_frac']}")

    baseline = None
    if not args.no_cpu_baseline:
        log("timing the NumPy oracle on the host (bounded sample)")
        baseline = cpu_baseline(config, weights, dtype, context, first_timed_position, args.cpu_steps)

    result = {
        "metric": METRIC,
        "value": round(decode_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random-init weights N(0,0.02), norms=1; uniform random prompt ids)",
        "config": {
            "workload": "C2: TinyLlama-1.1B-shape fp16 greedy decode, batch 1, 512-token prompt",
            "prompt": PROMPT, "context": context, "timed_positions": [int(positions[0]), int(positions[-1])],
            "decode_loop": "device-resident greedy (donated KV caches, no host round trip per token)",
            "kernels_per_token": program.kernel_count + 1,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "kernel": dominant, "bytes_per_launch": int(dom_bytes), "avg_launch_us": dom_us,
        },
        "cpu_baseline": baseline,
        "step_roofline": {"bytes_per_token": int(bytes_per_token), "achieved_gbps": round(step_gbps, 1),
                          "frac": round(step_gbps / HBM_PEAK_GBPS, 4)},
        "gpu_event_ms_per_step": round(gpu_ms.value / args.steps, 4),
        "prefill_tok_per_s": round(PROMPT / (prefill_ms * 1e-3), 1),
        "prefill_ms": {"stream_events": round(prefill_ms, 3), "host_wall": round(prefill_wall_ms, 2)},
        "prefill_c3": prefill_c3,
        "c4_batched_decode": c4,
        "c5_speculative": c5,
        "kernel_breakdown": breakdown,
        "first_tokens": tokens[:16],
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
