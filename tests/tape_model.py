"""Host model of a plan tape -- TEST INFRASTRUCTURE ONLY.

Decodes the int64 tape that ``chomikgrad._planner`` emits for
``chip_plan_create`` and executes each step with NumPy, following the kernel
semantics documented in chomik-grad_amd/csrc/*.hip (same parameter layout,
same rounding points).  It lets CPU tests check the planner's lowering,
fusion, memory plan and tape encoding against the oracle without a GPU.  It
is never used by the product.

``CpuPlanCompiler`` is a ``HIPCompiler`` whose device hands out host arrays
with fake device addresses, so ``plan_graph`` runs unchanged.
"""

from __future__ import annotations

import itertools
from typing import Dict, List

import numpy as np

from chomikgrad import _planner as P
from chomikgrad.dtypes import BFLOAT16
from chomikgrad.hip_backend import HIPCompiler

_addresses = itertools.count(1 << 24, 1 << 12)

DT = {0: np.dtype(np.float32), 1: np.dtype(np.float16), 2: np.dtype(np.uint16),
      3: np.dtype(np.int32), 4: np.dtype(np.int64)}


class HostArray:
    def __init__(self, host: np.ndarray):
        self.host = np.ascontiguousarray(host)
        self.shape = self.host.shape
        self.dtype = self.host.dtype
        self.nbytes = self.host.nbytes
        self.ptr = next(_addresses)


class HostDevice:
    name = "hip"

    def array(self, value):
        return value if isinstance(value, HostArray) else HostArray(np.asarray(value))

    def zeros(self, shape, dtype):
        return HostArray(np.zeros(shape, dtype))


class CpuPlanCompiler(HIPCompiler):
    def __init__(self):  # no library, no GPU
        self.device = HostDevice()
        self._rope_tables = {}
        self._program_cache = {}


def _round(values: np.ndarray, code: int) -> np.ndarray:
    values = np.asarray(values, dtype=np.float32)
    if code == 1:
        return values.astype(np.float16).astype(np.float32)
    if code == 2:
        return _bf16_to_f32(_f32_to_bf16(values))
    return values


def _f32_to_bf16(values: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    return np.where(nan, np.uint16(0x7FC0), rounded)


def _bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


class Memory:
    def __init__(self, planned: P.PlannedProgram, inputs: Dict, outputs: Dict):
        self.slots: Dict[int, np.ndarray] = {0: np.zeros(max(planned.arena_bytes, 16), np.uint8)}
        for storage in planned.storages:
            if storage.slot <= 0:
                continue
            if storage.kind == "const":
                self.slots[storage.slot] = storage.native.host.view(np.uint8).reshape(-1).copy()
            elif storage.kind == "input":
                self.slots[storage.slot] = inputs[storage.leaf]
            elif storage.kind == "output":
                self.slots[storage.slot] = outputs[id(storage)]

    def view(self, ptr, code, count) -> np.ndarray:
        slot, offset = ptr
        buffer = self.slots[slot]
        dtype = DT[code]
        return np.ndarray((count,), dtype=dtype, buffer=buffer, offset=offset)

    def flat(self, ptr, code) -> np.ndarray:
        slot, offset = ptr
        buffer = self.slots[slot]
        dtype = DT[code]
        return np.ndarray(((buffer.size - offset) // dtype.itemsize,), dtype=dtype, buffer=buffer, offset=offset)


def load(mem: Memory, ptr, code, index) -> np.ndarray:
    data = mem.flat(ptr, code)[np.asarray(index, dtype=np.int64)]
    if code == 2:
        return _bf16_to_f32(data)
    return data.astype(np.float32)


def store(mem: Memory, ptr, code, index, values) -> None:
    target = mem.flat(ptr, code)
    values = np.asarray(values, dtype=np.float32)
    if code == 2:
        target[np.asarray(index, dtype=np.int64)] = _f32_to_bf16(values)
    else:
        target[np.asarray(index, dtype=np.int64)] = values.astype(DT[code])


def strided_index(sizes, strides) -> np.ndarray:
    index = np.zeros([int(s) for s in sizes], dtype=np.int64)
    for d, (size, stride) in enumerate(zip(sizes, strides)):
        shape = [1] * len(sizes)
        shape[d] = int(size)
        index = index + np.arange(int(size), dtype=np.int64).reshape(shape) * int(stride)
    return index.reshape(-1) if len(sizes) else np.zeros(1, dtype=np.int64)


def decode(tape: np.ndarray):
    words = [int(w) for w in tape]
    assert words[0] == 0x43484950 and words[1] == 1
    n_steps = words[3]
    at = 5
    steps = []
    for _ in range(n_steps):
        kind, n_ptr, n_int, n_float = words[at:at + 4]
        at += 4
        ptrs = [(words[at + 2 * i], words[at + 2 * i + 1]) for i in range(n_ptr)]
        at += 2 * n_ptr
        ints = words[at:at + n_int]
        at += n_int
        floats = [float(np.array([w], dtype=np.uint32).view(np.float32)[0]) for w in words[at:at + n_float]]
        at += n_float
        steps.append((kind, ptrs, ints, floats))
    assert at == len(words)
    return steps


def run(planned: P.PlannedProgram, leaf_values: Dict) -> List[np.ndarray]:
    """Execute ``planned`` with host values for its input leaves."""
    inputs = {}
    for leaf, slot in planned.input_slots.items():
        value = np.asarray(leaf_values[leaf])
        if value.dtype == BFLOAT16:
            value = value.view(np.uint16)
        inputs[leaf] = np.ascontiguousarray(value).view(np.uint8).reshape(-1).copy()
    outputs = {}
    for kind, payload in planned.output_specs:
        if kind == "output" and id(payload) not in outputs:
            outputs[id(payload)] = np.zeros(max(payload.nbytes, 1), np.uint8)
    mem = Memory(planned, inputs, outputs)
    errors = 0
    for kind, ptrs, n, f in decode(planned.tape):
        errors |= STEP[kind](mem, ptrs, n, f)
    if errors:
        raise IndexError(f"kernel error bits {errors}")
    results = []
    for index, (kind, payload) in enumerate(planned.output_specs):
        node = planned.output_nodes[index]
        if kind == "output":
            raw = outputs[id(payload)][: payload.nbytes]
        elif kind == "input":
            raw = inputs[payload] if payload in inputs else np.ascontiguousarray(
                np.asarray(leaf_values[payload])).view(np.uint8).reshape(-1)
        elif kind == "const":
            raw = payload.host.view(np.uint8).reshape(-1)
        else:
            results.append(np.zeros(node.shape, node.dtype))
            continue
        dtype = np.dtype(np.uint16) if node.dtype == BFLOAT16 else node.dtype
        value = raw.view(dtype).reshape(node.shape).copy()
        results.append(value.view(BFLOAT16) if node.dtype == BFLOAT16 else value)
    return results


# ---------------------------------------------------------------- steps
def s_fill(mem, p, n, f):
    mem.view(p[0], 3, n[0])[:] = n[1]
    return 0


def s_copy(mem, p, n, f):
    count, nd = n[0], n[1]
    size = n[18]
    index = strided_index(n[2:2 + nd], n[10:10 + nd])
    target = strided_index(n[2:2 + nd], n[20:20 + nd]) if n[19] else np.arange(count)
    if size == 1:
        src = mem.slots[p[0][0]][p[0][1]:]
        mem.slots[p[1][0]][p[1][1] + target] = src[index]
        return 0
    code = {2: 2, 4: 3, 8: 4}[size]
    mem.flat(p[1], code)[target] = mem.flat(p[0], code)[index]
    return 0


def s_elementwise(mem, p, n, f):
    count, nd = n[0], n[1]
    sizes = n[2:2 + nd]
    n_in, n_ops, out_dt = n[10], n[11], n[12]
    regs = []
    for k in range(n_in):
        strides = n[19 + 8 * k: 19 + 8 * k + nd]
        regs.append(load(mem, p[1 + k], n[13 + k], strided_index(sizes, strides)))
    with np.errstate(all="ignore"):
        for o in range(n_ops):
            code = n[67 + o]
            op, a, b, rd = code & 0xFF, (code >> 8) & 0xFF, (code >> 16) & 0xFF, (code >> 24) & 0xFF
            x, y = regs[a], regs[b]
            v = {1: lambda: x + y, 2: lambda: x - y, 3: lambda: x * y, 4: lambda: x / y,
                 5: lambda: (x == y).astype(np.float32), 6: lambda: -x, 7: lambda: np.exp(x),
                 8: lambda: np.log(x), 9: lambda: np.sqrt(x), 10: lambda: np.maximum(x, 0),
                 11: lambda: (x > 0).astype(np.float32)}[op]()
            regs.append(_round(v, rd))
    store(mem, p[0], out_dt, np.arange(count), regs[-1])
    return 0


def s_reduce(mem, p, n, f):
    n_out, red_len, kind, in_dt, out_dt, nk = n[0:6]
    kept = strided_index(n[6:6 + nk], n[14:14 + nk])
    nr = n[22]
    red = strided_index(n[23:23 + nr], n[31:31 + nr])
    values = load(mem, p[0], in_dt, kept[:, None] + red[None, :])
    result = values.sum(axis=1) if kind == 0 else values.max(axis=1)
    store(mem, p[1], out_dt, np.arange(n_out), _round(result, out_dt))
    return 0


def s_gather(mem, p, n, f):
    n_ids, rows, row_bytes, id_dt = n[0:4]
    ids = mem.view(p[1], id_dt, n_ids).astype(np.int64)
    ids = np.where(ids < 0, ids + rows, ids)
    bad = (ids < 0) | (ids >= rows)
    table = mem.flat(p[0], 0).view(np.uint8)[: rows * row_bytes].reshape(rows, row_bytes)
    out = mem.flat(p[2], 0).view(np.uint8)[: n_ids * row_bytes].reshape(n_ids, row_bytes)
    out[:] = np.where(bad[:, None], 0, table[np.clip(ids, 0, rows - 1)])
    return 1 if bad.any() else 0


def s_matmul(mem, p, n, f):
    batch, M, N, K, adt, bdt, cdt, sam, sak, sbk, sbn, nb = n[0:12]
    bsizes = n[12:12 + nb]
    bidx_a = strided_index(bsizes, n[16:16 + nb])
    bidx_b = strided_index(bsizes, n[20:20 + nb])
    a_idx = bidx_a[:, None, None] + (np.arange(M)[:, None] * sam + np.arange(K)[None, :] * sak)[None]
    b_idx = bidx_b[:, None, None] + (np.arange(K)[:, None] * sbk + np.arange(N)[None, :] * sbn)[None]
    A = load(mem, p[0], adt, a_idx)
    B = load(mem, p[1], bdt, b_idx)
    C = np.matmul(A.astype(np.float64), B.astype(np.float64)).astype(np.float32)
    store(mem, p[2], cdt, np.arange(batch * M * N), _round(C.reshape(-1), cdt))
    return 0


def s_softmax(mem, p, n, f):
    rows, length, dt, is_, os_, nk = n[0:6]
    kin = strided_index(n[6:6 + nk], n[14:14 + nk])
    kout = strided_index(n[6:6 + nk], n[22:22 + nk])
    x = load(mem, p[0], dt, kin[:, None] + np.arange(length)[None, :] * is_)
    with np.errstate(all="ignore"):
        e = _round(np.exp(_round(x - x.max(axis=1, keepdims=True), dt)), dt)
        s = _round(e.sum(axis=1, keepdims=True), dt)
        y = _round(e / s, dt)
    store(mem, p[1], dt, (kout[:, None] + np.arange(length)[None, :] * os_).reshape(-1), y.reshape(-1))
    return 0


def _rms(x, w, eps, dt):
    ss = _round(_round(x * x, dt).sum(axis=-1, keepdims=True), dt)
    mean = _round(ss / _round(np.float32(x.shape[-1]), dt), dt)
    r = _round(np.sqrt(_round(mean + _round(np.float32(eps), dt), dt)), dt)
    return _round(_round(x / r, dt) * w, dt)


def s_rmsnorm(mem, p, n, f):
    rows, D, rs, dt, wdt = n[0:5]
    x = load(mem, p[0], dt, np.arange(rows)[:, None] * rs + np.arange(D)[None, :])
    w = load(mem, p[1], wdt, np.arange(D))
    store(mem, p[2], dt, np.arange(rows * D), _rms(x, w, f[0], dt).reshape(-1))
    return 0


def s_rope(mem, p, n, f):
    B, H, T, hd = n[0:4]
    xs = n[4:8]
    dt, mode, offset, length = n[8:12]
    half = hd // 2
    error = 0
    out = np.zeros((B, H, T, hd), np.float32)
    for b in range(B):
        for t in range(T):
            pos = offset + t
            if mode == 1:
                pos += int(mem.view(p[1], 3, 1)[0])
            if mode == 2:
                pos += int(mem.view(p[1], 3, B)[b])
            if not 0 <= pos < length:
                error |= 2
                continue
            c = load(mem, p[2], dt, pos * hd + np.arange(half))
            s = load(mem, p[2], dt, pos * hd + half + np.arange(half))
            for h in range(H):
                base = b * xs[0] + h * xs[1] + t * xs[2]
                x1 = load(mem, p[0], dt, base + np.arange(half) * xs[3])
                x2 = load(mem, p[0], dt, base + (np.arange(half) + half) * xs[3])
                out[b, h, t, :half] = x1 * c + x2 * -s
                out[b, h, t, half:] = x1 * s + x2 * c
    store(mem, p[3], dt, np.arange(out.size), out.reshape(-1))
    return error


def s_sdpa(mem, p, n, f):
    B, H, T, C, hd, KV, dt = n[0:7]
    qs, ks, vs, ms = n[7:11], n[11:15], n[15:19], n[19:23]
    mdt = n[23]
    div = _round(np.float32(f[0]), dt)
    out = np.zeros((B, H, T, hd), np.float32)
    with np.errstate(all="ignore"):
        for b in range(B):
            for h in range(H):
                g = h // (H // KV)
                K = load(mem, p[1], dt, b * ks[0] + g * ks[1] + np.arange(C)[:, None] * ks[2] + np.arange(hd)[None, :] * ks[3])
                V = load(mem, p[2], dt, b * vs[0] + g * vs[1] + np.arange(C)[:, None] * vs[2] + np.arange(hd)[None, :] * vs[3])
                for t in range(T):
                    q = load(mem, p[0], dt, b * qs[0] + h * qs[1] + t * qs[2] + np.arange(hd) * qs[3])
                    s = _round(_round((K.astype(np.float64) @ q).astype(np.float32), dt) / div, dt)
                    if p[3][0] >= 0:
                        m = load(mem, p[3], mdt, b * ms[0] + h * ms[1] + t * ms[2] + np.arange(C) * ms[3])
                        s = _round(s + m, dt)
                    e = _round(np.exp(_round(s - s.max(), dt)), dt)
                    S = _round(e.sum(), dt)
                    out[b, h, t] = (_round(e / S, dt).astype(np.float64) @ V).astype(np.float32)
    o = n[26:29]
    index = (np.arange(B)[:, None, None, None] * o[0] + np.arange(H)[None, :, None, None] * o[1]
             + np.arange(T)[None, None, :, None] * o[2] + np.arange(hd)[None, None, None, :])
    store(mem, p[4], dt, index.reshape(-1), out.reshape(-1))
    return 0


def _blend(c, x, w, dt):
    return _round(_round(c * _round(1 - w, dt), dt) + _round(x * w, dt), dt)


def s_kv_write(mem, p, n, f):
    B, KV, C, hd, dt = n[0:5]
    xs = n[5:9]
    wsb, wsr, in_place = n[9:12]
    cs = n[12:16]
    wdt = n[16]
    for b in range(B):
        w = load(mem, p[2], wdt, b * wsb + np.arange(C) * wsr)
        for g in range(KV):
            cidx = b * cs[0] + g * cs[1] + np.arange(C)[:, None] * cs[2] + np.arange(hd)[None, :] * cs[3]
            xidx = b * xs[0] + g * xs[1] + np.arange(C)[:, None] * xs[2] + np.arange(hd)[None, :] * xs[3]
            c = load(mem, p[0], dt, cidx)
            x = load(mem, p[1], dt, xidx)
            new = _blend(c, x, w[:, None], dt)
            if in_place:
                rows = w != 0
                store(mem, p[3], dt, cidx[rows].reshape(-1), new[rows].reshape(-1))
            else:
                base = ((b * KV + g) * C) * hd
                store(mem, p[3], dt, base + np.arange(C * hd), new.reshape(-1))
    return 0


def s_kv_place(mem, p, n, f):
    B, KV, C, hd, dt, T = n[0:6]
    pls = n[10:12]
    wsb, wsr, in_place = n[12:15]
    cs = n[15:19]
    pdt, wdt = n[19:21]
    pair, rope = n[21] if len(n) > 21 else 0, n[26] if len(n) > 26 else 0
    assert not pair or (p[5][0] >= 0 and p[6][0] >= 0 and p[7][0] >= 0 and p[8][0] >= 0), "paired kv_place unbound"
    pl = load(mem, p[2], pdt, np.arange(T)[:, None] * pls[0] + np.arange(C)[None, :] * pls[1])
    error = 0
    members = [(p[0], p[1], p[4], n[6:10], bool(rope))]
    if pair:
        members.append((p[5], p[6], p[7], n[22:26], False))
    for cache_p, x_p, out_p, xs, rotate in members:
        for b in range(B):
            w = load(mem, p[3], wdt, b * wsb + np.arange(C) * wsr)
            touched = (w != 0) | (pl != 0).any(axis=0)
            for g in range(KV):
                x = load(mem, x_p, dt, b * xs[0] + g * xs[1] + np.arange(T)[:, None] * xs[2] + np.arange(hd)[None, :] * xs[3])
                if rotate:
                    # the keys' RoPE on load (k_rope's arithmetic, rounded once)
                    half = hd // 2
                    pos = n[28] + np.arange(T) + (int(mem.view(p[9], 3, 1)[0]) if n[27] == 1 else 0)
                    ok = (pos >= 0) & (pos < n[29])
                    if not ok.all():
                        error |= 2
                    safe = np.where(ok, pos, 0)
                    c = load(mem, p[8], dt, safe[:, None] * hd + np.arange(half)[None, :])
                    s = load(mem, p[8], dt, safe[:, None] * hd + half + np.arange(half)[None, :])
                    x1, x2 = x[:, :half], x[:, half:]
                    x = _round(np.concatenate([x1 * c + x2 * -s, x1 * s + x2 * c], axis=1), dt)
                    x[~ok] = 0
                placed = _round((pl.T.astype(np.float64) @ x).astype(np.float32), dt)
                cidx = b * cs[0] + g * cs[1] + np.arange(C)[:, None] * cs[2] + np.arange(hd)[None, :] * cs[3]
                c = load(mem, cache_p, dt, cidx)
                new = _round(_round(c * _round(1 - w[:, None], dt), dt) + placed, dt)
                if in_place:
                    store(mem, out_p, dt, cidx[touched].reshape(-1), new[touched].reshape(-1))
                else:
                    store(mem, out_p, dt, ((b * KV + g) * C) * hd + np.arange(C * hd), new.reshape(-1))
    return error


def s_gemv(mem, p, n, f):
    M, K, xs, dt, nseg, pro, silu = n[0:7]
    # a GEMV split over blocks needs its bound workspace (tickets, partials)
    assert n[24] <= 1 or (p[14][0] >= 0 and n[25] >= 4 * -(-max(n[7:11]) // 16)), "split GEMV without a workspace"
    Ns = n[7:11]
    ostr = n[11:15]
    rstr = n[15:19]
    wdt = n[19]
    x = load(mem, p[0], dt, np.arange(M)[:, None] * xs + np.arange(K)[None, :])
    if pro:
        x = _rms(x, load(mem, p[1], wdt, np.arange(K)), f[0], dt)
    with np.errstate(all="ignore"):
        if silu:
            N = Ns[0]
            g = _round((x.astype(np.float64) @ load(mem, p[2], dt, np.arange(N)[:, None] * K + np.arange(K)[None, :]).T.astype(np.float64)).astype(np.float32), dt)
            u = _round((x.astype(np.float64) @ load(mem, p[3], dt, np.arange(N)[:, None] * K + np.arange(K)[None, :]).T.astype(np.float64)).astype(np.float32), dt)
            act = _round(_round(g / _round(_round(np.exp(-g), dt) + 1, dt), dt) * u, dt)
            store(mem, p[6], dt, (np.arange(M)[:, None] * ostr[0] + np.arange(N)[None, :]).reshape(-1), act.reshape(-1))
            return 0
        for s in range(nseg):
            N = Ns[s]
            W = load(mem, p[2 + s], dt, np.arange(N)[:, None] * K + np.arange(K)[None, :])
            y = _round((x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32), dt)
            if p[10 + s][0] >= 0:
                res = load(mem, p[10 + s], dt, np.arange(M)[:, None] * rstr[s] + np.arange(N)[None, :])
                y = _round(res + y, dt)
            store(mem, p[6 + s], dt, (np.arange(M)[:, None] * ostr[s] + np.arange(N)[None, :]).reshape(-1), y.reshape(-1))
    return 0


def s_attn_proj(mem, p, n, f):
    """Combine of the decode attention's partials (batch 1), then the output
    projection y = round(r + round(W x)) of the combined x."""
    N, K, H, NS, dt = n[0:5]
    assert K == 64 * H and 2 <= NS <= 32
    total = H * NS
    parts = mem.view(p[0], 0, total * 66).astype(np.float64)
    O = parts[:total * 64].reshape(H, NS, 64)
    m = parts[total * 64:total * 65].reshape(H, NS)
    s = parts[total * 65:].reshape(H, NS)
    with np.errstate(all="ignore"):
        f = np.exp(m - m.max(axis=1, keepdims=True))
        fac = f / (s * f).sum(axis=1, keepdims=True)
        x = _round((O * fac[:, :, None]).sum(axis=1).astype(np.float32), dt).reshape(1, K)
        W = load(mem, p[1], dt, np.arange(N)[:, None] * K + np.arange(K)[None, :])
        y = _round((x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32), dt)
        if p[2][0] >= 0:
            y = _round(load(mem, p[2], dt, np.arange(N)[None, :]) + y, dt)
    store(mem, p[3], dt, np.arange(N), y.reshape(-1))
    return 0


def s_gemm(mem, p, n, f):
    M, N, K, dt, lda, ldw, ldc, ldr, silu, ldwu, has_res = n[0:11]
    A = load(mem, p[0], dt, np.arange(M)[:, None] * lda + np.arange(K)[None, :])
    if n[11] > 1:  # output segments: sibling products of A
        assert not silu and not has_res and sum(n[12:12 + n[11]]) == N
        wp = [p[1]] + [p[5 + 2 * k] for k in range(n[11] - 1)]
        cp = [p[2]] + [p[6 + 2 * k] for k in range(n[11] - 1)]
        for s in range(n[11]):
            Ns, lc, lw = n[12 + s], n[16 + s], n[20 + s]
            assert Ns % 128 == 0
            W = load(mem, wp[s], dt, np.arange(Ns)[:, None] * lw + np.arange(K)[None, :])
            C = _round((A.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32), dt)
            store(mem, cp[s], dt, (np.arange(M)[:, None] * lc + np.arange(Ns)[None, :]).reshape(-1), C.reshape(-1))
        return 0
    W = load(mem, p[1], dt, np.arange(N)[:, None] * ldw + np.arange(K)[None, :])
    C = _round((A.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32), dt)
    if silu:  # C = round(silu(round(g)) * round(u)), silu(g) = round(g / round(round(exp(-g)) + 1))
        Wu = load(mem, p[4], dt, np.arange(N)[:, None] * ldwu + np.arange(K)[None, :])
        U = _round((A.astype(np.float64) @ Wu.T.astype(np.float64)).astype(np.float32), dt)
        with np.errstate(over="ignore"):
            denom = _round(_round(np.exp(-C), dt) + 1, dt)
        C = _round(_round(C / denom, dt) * U, dt)
    elif has_res:  # residual epilogue
        R = load(mem, p[3], dt, np.arange(M)[:, None] * ldr + np.arange(N)[None, :])
        C = _round(R + C, dt)
    store(mem, p[2], dt, (np.arange(M)[:, None] * ldc + np.arange(N)[None, :]).reshape(-1), C.reshape(-1))
    return 0


def s_decode_attn(mem, p, n, f):
    B, H, KV, C, dt = n[0:5]
    qs, ks, vs = n[5:8], n[8:11], n[11:14]
    mode, length = n[14], n[15]
    cs = n[16:20]
    wsb, wsc, msb, msh, msc, mdt, wdt, in_place, passes, stream_rows, unroll, partials_only, read_only = n[20:33]
    # read only: T query rows of one block over one already-updated cache
    # (cache batch stride 0, positions position[0] + b, nothing written but
    # the output); only on the chunk kernel
    assert not read_only or (passes in (1, 2, 4) and mode == 3 and cs[0] == 0 and not partials_only)
    assert (passes in (1, 2, 4) or (passes == 0 and stream_rows > 0 and unroll in (2, 4))
            or (passes == 8 and dt in (1, 2) and 1 <= stream_rows <= 3 and -(-C // 32) <= 8 * stream_rows))
    rpp = 16 if dt == 0 else 32
    chunks = 1 if passes == 8 else -(-C // stream_rows) if passes == 0 else -(-C // (rpp * passes))
    assert chunks <= 64 and (passes != 0 or stream_rows % rpp == 0)
    assert not partials_only or (passes in (1, 2, 4) and chunks >= 2 and B == 1)
    if partials_only:
        # partials that combine to the output: chunk 0 holds it with maximum
        # 0 and exp-sum 1, the other chunks maximum -inf and exp-sum 0
        total = H * chunks
        parts = mem.view(p[13], 0, total * 66)
        parts[:] = 0.0
        parts[total * 64:total * 65].reshape(H, chunks)[:, 1:] = -np.inf
        parts[total * 65:total * 66].reshape(H, chunks)[:, 0] = 1.0
    G = H // KV
    div = _round(np.float32(f[0]), dt)
    error = 0
    d = np.arange(64)
    newk = {}
    for b in range(B):
        pos = int(mem.view(p[3], 3, B if mode == 2 else 1)[b if mode == 2 else 0]) + (b if mode == 3 else 0)
        if not 0 <= pos < length:
            error |= 2
            pos = 0
        c = load(mem, p[4], dt, pos * 64 + np.arange(32))
        s = load(mem, p[4], dt, pos * 64 + 32 + np.arange(32))

        def rope(x):
            return _round(np.concatenate([x[:32] * c + x[32:] * -s, x[:32] * s + x[32:] * c]), dt)

        w = np.zeros(C, np.float32) if read_only else load(mem, p[7], wdt, b * wsb + np.arange(C) * wsc)
        keep = _round(1 - w, dt)[:, None]
        for g in range(KV):
            if read_only:
                k = v = np.zeros(64, np.float32)
            else:
                k = rope(load(mem, p[1], dt, b * ks[0] + g * ks[1] + d * ks[2]))
                v = load(mem, p[2], dt, b * vs[0] + g * vs[1] + d * vs[2])
            idx = b * cs[0] + g * cs[1] + np.arange(C)[:, None] * cs[2] + d[None, :] * cs[3]
            Kc, Vc = load(mem, p[5], dt, idx), load(mem, p[6], dt, idx)
            Kn = np.where(w[:, None] != 0, _round(_round(Kc * keep, dt) + _round(k[None] * w[:, None], dt), dt), Kc)
            Vn = np.where(w[:, None] != 0, _round(_round(Vc * keep, dt) + _round(v[None] * w[:, None], dt), dt), Vc)
            newk[(b, g)] = (idx, Kn, Vn, w)
            with np.errstate(all="ignore"):
                for h in range(g * G, (g + 1) * G):
                    q = rope(load(mem, p[0], dt, b * qs[0] + h * qs[1] + d * qs[2]))
                    sc = _round(_round((Kn.astype(np.float64) @ q).astype(np.float32), dt) / div, dt)
                    if p[8][0] >= 0:
                        sc = _round(sc + load(mem, p[8], mdt, b * msb + h * msh + np.arange(C) * msc), dt)
                    # float32 softmax and P V (one division, one rounding)
                    e = np.exp(sc.astype(np.float64) - np.float64(sc.max()))
                    out = ((e @ Vn.astype(np.float64)) / e.sum()).astype(np.float32)
                    if partials_only:
                        parts[(h * chunks) * 64 + d] = out
                    else:
                        store(mem, p[9], dt, (b * H + h) * 64 + d, out)
    for (b, g), (idx, Kn, Vn, w) in newk.items():
        if read_only:
            continue
        if in_place:
            rows = w != 0
            store(mem, p[10], dt, idx[rows].reshape(-1), Kn[rows].reshape(-1))
            store(mem, p[11], dt, idx[rows].reshape(-1), Vn[rows].reshape(-1))
        else:
            base = ((b * KV + g) * C) * 64
            store(mem, p[10], dt, base + np.arange(C * 64), Kn.reshape(-1))
            store(mem, p[11], dt, base + np.arange(C * 64), Vn.reshape(-1))
    return error


STEP = {
    P.K_FILL: s_fill, P.K_COPY: s_copy, P.K_ELEMENTWISE: s_elementwise, P.K_REDUCE: s_reduce,
    P.K_GATHER: s_gather, P.K_MATMUL: s_matmul, P.K_SOFTMAX: s_softmax, P.K_RMSNORM: s_rmsnorm,
    P.K_ROPE: s_rope, P.K_SDPA: s_sdpa, P.K_KV_WRITE: s_kv_write, P.K_KV_PLACE: s_kv_place,
    P.K_GEMV: s_gemv, P.K_GEMM: s_gemm, P.K_DECODE_ATTN: s_decode_attn, P.K_ATTN_PROJ: s_attn_proj,
}
