"""Backend-local planning for the ``hip`` plugin.

``plan_graph`` turns the output nodes of a lazy graph into a flat list of
kernel steps over planned buffers, then serialises it as the int64 tape that
``chip_plan_create`` (include/chomik_hip.h) executes as one hipGraph.

Stages
1. Lowering choice (never mutating a ``LazyNode``; reference rule,
   chomikgrad/lazy.py:252-264): the intrinsic tags ``rms_norm``, ``rope``,
   ``sdpa`` and ``softmax`` when their operands fit a kernel, plus
   plugin-local rewrites of portable patterns:
     linear    MATMUL(x, PERMUTE(W, (1, 0)))                  llama.py _linear
     kv_write  c * (1 - w) + x * w                            llama.py:511-512
     kv_place  c * (1 - w) + PERMUTE(MATMUL(PERMUTE(x), P))   llama.py:633-640
     silu_mul  (g / (1 + exp(-g))) * u                        llama.py _silu/_mlp
   then single-consumer ELEMENTWISE chains are fused (GraphPlan).
2. Emission: one step per remaining node; RESHAPE/PERMUTE become strided
   views whenever the data allows.
3. Step fusion: RMSNorm into the prologue of the GEMVs that consume it,
   gate/up GEMVs + SiLU into one dual-weight GEMV, sibling GEMVs sharing an
   input into one multi-segment launch, and residual adds into the GEMV
   epilogue.
4. Memory: intermediates share one arena by liveness; program outputs get
   caller-visible buffers; donated KV caches are updated in place.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Set, Tuple

import numpy as np

from .dtypes import BFLOAT16, dtype_code, dtype_name, is_float, is_integer
from .lazy import GraphPlan, LazyNode, Op, op_of

# Step kinds (enum chip_kind in include/chomik_hip.h).
K_FILL, K_COPY, K_ELEMENTWISE, K_REDUCE, K_GATHER, K_MATMUL, K_SOFTMAX = 1, 2, 3, 4, 5, 6, 7
K_RMSNORM, K_ROPE, K_SDPA, K_KV_WRITE, K_KV_PLACE, K_GEMV, K_GEMM = 8, 9, 10, 11, 12, 13, 14
K_DECODE_ATTN = 17
K_ATTN_PROJ = 18

KIND_NAMES = {
    K_FILL: "fill", K_COPY: "copy", K_ELEMENTWISE: "fused_elementwise",
    K_REDUCE: "reduce", K_GATHER: "gather", K_MATMUL: "matmul", K_SOFTMAX: "softmax",
    K_RMSNORM: "rms_norm", K_ROPE: "rope", K_SDPA: "sdpa", K_KV_WRITE: "kv_write",
    K_KV_PLACE: "kv_place", K_GEMV: "gemv", K_GEMM: "gemm", K_DECODE_ATTN: "decode_attention",
    K_ATTN_PROJ: "attn_proj",
}

OPCODES = {"add": 1, "sub": 2, "mul": 3, "div": 4, "equal": 5, "neg": 6, "exp": 7,
           "log": 8, "sqrt": 9, "relu": 10, "step": 11}
MAX_DIMS = 8
MAX_EW_INPUTS = 6
MAX_EW_OPS = 24
GEMV_MAX_ROWS = 8
GEMV_STAGE_BYTES = 48 * 1024
# batches of 2..8 independent rows on the row-exact kernels where they beat
# the MFMA kernel (lower_linear); 0 keeps every batch GEMV on MFMA
GEMV_BATCH_ROW_EXACT = os.environ.get("CHOMIK_HIP_GEMV_BATCH_ROW_EXACT", "1") != "0"
GEMV_BATCH_ROW_EXACT_MAX_K = int(os.environ.get("CHOMIK_HIP_GEMV_BATCH_ROW_EXACT_MAX_K", "2048"))
# Waves sharing one GEMV row group (K split): 0 lets the kernel choose from
# the row count; CHOMIK_HIP_GEMV_SPLIT=1/2/4 forces one (for tuning sweeps).
GEMV_SPLIT = int(os.environ.get("CHOMIK_HIP_GEMV_SPLIT", "0"))
# Decode attention (cache rows per pass: 32 for 2-byte, 16 for 4-byte
# dtypes): 0 chooses; 1, 2 or 4 force the chunk kernel with that
# many passes per workgroup; -1 forces the streaming kernel; -2 the MFMA
# kernel where it applies (16-bit caches of at most 768 rows; one workgroup
# per KV head, measured slower than the chunk kernel at the C2 shape: one CU
# keeps too few HBM misses in flight for 160 KB, so it is never chosen).
DECODE_ATTN_PASSES = int(os.environ.get("CHOMIK_HIP_ATTN_PASSES", "0"))
DECODE_ATTN_MAX_CHUNKS = 64
# The streaming kernel takes over when the chunk kernel would need more than
# this many workgroups (several latency-bound rounds); it launches about
# DECODE_ATTN_STREAM_WGS workgroups with DECODE_ATTN_STREAM_UNROLL passes
# per tile (2 or 4; 2 measured faster at batch 8 over 4096 cached rows).  At
# batch 8 x 8 KV heads over 4096 rows, 512 workgroups (two per CU, 512 rows
# each) measured 0.8 % faster than 768 or 640, and 384 or 256 slower.
DECODE_ATTN_STREAM_ABOVE = int(os.environ.get("CHOMIK_HIP_ATTN_STREAM_ABOVE", "768"))
DECODE_ATTN_STREAM_WGS = int(os.environ.get("CHOMIK_HIP_ATTN_STREAM_WGS", "512"))
DECODE_ATTN_STREAM_UNROLL = int(os.environ.get("CHOMIK_HIP_ATTN_STREAM_UNROLL", "2"))
# Batch-1 decode, opt-in: the chunk attention stores only its partials and
# the output projection (the next GEMV) combines them instead of the
# attention's own cross-workgroup ticket and combine.  Measured at the C2
# shape it loses (attention 8.9 -> 5.6 us, but the projection 4.0 -> 8.2 us:
# each block reads every head's partials, 169 KB, before its dot products),
# so it is off by default.
ATTN_PROJ_FUSE = int(os.environ.get("CHOMIK_HIP_ATTN_PROJ", "0"))
ATTN_PROJ_MAX_CHUNKS = 32
# The MFMA kernel: one workgroup of at most 8 waves per (sequence, KV head),
# each wave with 1-3 blocks of 32 cache rows in registers.
DECODE_ATTN_MFMA_BLOCK = 32
DECODE_ATTN_MFMA_WAVES = 8
DECODE_ATTN_MFMA_MAX_BLOCKS = 3
SDPA_MAX_KEYS = 32768
ARENA_ALIGN = 256
SUPPORTED_TAGS = frozenset({"rms_norm", "rope", "sdpa", "softmax"})


class PlanError(NotImplementedError):
    """A node the hip plugin cannot execute (raised at compile time)."""


def contiguous_strides(shape: Sequence[int]) -> Tuple[int, ...]:
    strides = []
    running = 1
    for size in reversed(shape):
        strides.append(running)
        running *= max(int(size), 1)
    return tuple(reversed(strides))


def _prod(values: Sequence[int]) -> int:
    result = 1
    for value in values:
        result *= int(value)
    return result


# ---------------------------------------------------------------- buffers
class Storage:
    """A buffer: arena region, captured constant, program input or output."""

    __slots__ = ("kind", "nbytes", "leaf", "native", "slot", "offset", "first", "last", "label")

    def __init__(self, kind: str, nbytes: int, *, leaf=None, native=None, label=""):
        self.kind = kind
        self.nbytes = int(nbytes)
        self.leaf = leaf
        self.native = native
        self.slot = -1
        self.offset = 0
        self.first = -1
        self.last = -1
        self.label = label


class PV:
    """A planned value: a (possibly strided) view of a storage."""

    __slots__ = ("shape", "dtype", "strides", "storage", "offset")

    def __init__(self, shape, dtype, strides, storage: Storage, offset: int = 0):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.strides = tuple(int(s) for s in strides)
        self.storage = storage
        self.offset = int(offset)

    @property
    def size(self) -> int:
        return _prod(self.shape)

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    def contiguous(self) -> bool:
        expected = contiguous_strides(self.shape)
        return all(size == 1 or a == b for size, a, b in zip(self.shape, self.strides, expected))

    def whole(self) -> bool:
        """Contiguous and covering its whole storage from offset 0."""
        return self.contiguous() and self.offset == 0 and self.size * self.itemsize == self.storage.nbytes

    def same_data(self, other: "PV") -> bool:
        return (self.storage is other.storage and self.offset == other.offset
                and self.size == other.size and self.contiguous() and other.contiguous())

    def row_stride(self) -> Optional[int]:
        """Stride between rows when viewed as (prod(shape[:-1]), shape[-1])
        with unit stride along the last axis, else None."""
        if not self.shape:
            return 1
        if self.shape[-1] != 1 and self.strides[-1] != 1:
            return None
        lead = [(s, st) for s, st in zip(self.shape[:-1], self.strides[:-1]) if s != 1]
        if not lead:
            return self.shape[-1]
        for (size_a, stride_a), (size_b, stride_b) in zip(lead, lead[1:]):
            if stride_a != stride_b * size_b:
                return None
        return lead[-1][1]


@dataclass
class Step:
    kind: int
    ins: List[PV]
    outs: List[PV]
    attrs: Dict[str, object] = field(default_factory=dict)

    def reads(self) -> List[PV]:
        """Every value the step's kernel reads (for liveness and slots)."""
        if self.kind == K_GEMV:
            prologue = self.attrs["prologue"]
            values = [prologue["x"], prologue["w"]] if prologue else [self.ins[0]]
            for segment in self.attrs["segments"]:
                values.append(segment["w"])
                if segment["res"] is not None:
                    values.append(segment["res"])
            if self.attrs.get("workspace") is not None:  # split MFMA GEMV: tickets and partials
                values.append(self.attrs["workspace"])
            return values
        return [pv for pv in self.ins if pv is not None]


# ---------------------------------------------------------------- patterns
class _HipGraphPlan(GraphPlan):
    """GraphPlan that can also refuse an intrinsic tag for one node."""

    def __init__(self, outputs, supported):
        super().__init__(outputs, supported)
        self.refused: Set[LazyNode] = set()

    def lowering(self, node):
        if node in self.refused and node not in self._overrides:
            return None
        return super().lowering(node)


def _is_ew(node: LazyNode, kind: str) -> bool:
    return op_of(node) is Op.ELEMENTWISE and node.arg == kind


def _is_one(node: LazyNode, dynamic: Set[LazyNode]) -> bool:
    if node.op is not None or node in dynamic or node.value is None:
        return False
    value = np.asarray(node.value)
    if value.size == 0:
        return False
    if value.dtype == BFLOAT16:
        return bool(np.all(value.view(np.uint16) == 0x3F80))
    if not (is_float(value.dtype) or is_integer(value.dtype)):
        return False
    return bool(np.all(value == 1))


def _match_linear(node: LazyNode):
    if op_of(node) is not Op.MATMUL:
        return None
    a, b = node.inputs
    if op_of(b) is Op.PERMUTE and b.arg == (1, 0) and len(b.inputs[0].shape) == 2:
        return a, b.inputs[0]
    return None


def _match_one_minus(node: LazyNode, dynamic):
    if _is_ew(node, "sub") and _is_one(node.inputs[0], dynamic):
        return node.inputs[1]
    return None


def _match_kv_update(node: LazyNode, dynamic):
    """``c * (1 - w) + x * w`` -> ("kv_write", c, x, w) or
    ``c * (1 - w) + PERMUTE(MATMUL(PERMUTE(x), P))`` -> ("kv_place", ...)."""
    if not _is_ew(node, "add") or len(node.shape) != 4:
        return None
    kept, added = node.inputs
    if not _is_ew(kept, "mul"):
        return None
    cache, one_minus = kept.inputs
    w = _match_one_minus(one_minus, dynamic)
    if w is None or cache.shape != node.shape:
        return None
    if _is_ew(added, "mul") and added.inputs[1] is w:
        return ("kv_write", cache, added.inputs[0], w)
    if (op_of(added) is Op.PERMUTE and added.arg == (0, 1, 3, 2)
            and op_of(added.inputs[0]) is Op.MATMUL):
        inner, placement = added.inputs[0].inputs
        if (op_of(inner) is Op.PERMUTE and inner.arg == (0, 1, 3, 2)
                and len(placement.shape) == 2):
            return ("kv_place", cache, inner.inputs[0], placement, w)
    return None


def _match_silu_mul(node: LazyNode, dynamic):
    """``(g / (1 + exp(-g))) * u`` as built by llama.py _silu and _mlp."""
    if not _is_ew(node, "mul"):
        return None
    gated, up = node.inputs
    if not _is_ew(gated, "div"):
        return None
    g, denominator = gated.inputs
    if not _is_ew(denominator, "add"):
        return None
    exp_node, one = denominator.inputs
    if not (_is_one(one, dynamic) and _is_ew(exp_node, "exp")):
        return None
    neg = exp_node.inputs[0]
    if not (_is_ew(neg, "neg") and neg.inputs[0] is g):
        return None
    if g.shape != node.shape or up.shape != node.shape:
        return None
    return g, up, one


def _same_float_dtype(*nodes: LazyNode) -> bool:
    dtypes = {node.dtype for node in nodes}
    return len(dtypes) == 1 and is_float(next(iter(dtypes))) and next(iter(dtypes)) != np.float64


def choose_lowerings(outputs: Sequence[LazyNode], dynamic: Set[LazyNode]) -> _HipGraphPlan:
    plan = _HipGraphPlan(outputs, SUPPORTED_TAGS)
    # Refuse tags whose operands do not fit the fused kernels.
    for node in topological_nodes(plan):
        tag = node.lowering
        if tag is None or tag[0] not in SUPPORTED_TAGS:
            continue
        if not _tag_fits(node, tag):
            plan.refused.add(node)
    # Plugin-local rewrites; repeat until the rewritten graph is stable.
    changed = True
    while changed:
        changed = False
        for node in plan.nodes():
            if node.op is None or plan.lowering(node) is not None:
                continue
            rewrite = _rewrite(node, dynamic)
            if rewrite is not None:
                plan.override(node, rewrite)
                changed = True
    plan.fuse_elementwise()
    return plan


def topological_nodes(plan: GraphPlan):
    return plan.nodes()


def _rewrite(node: LazyNode, dynamic):
    linear = _match_linear(node)
    if linear is not None:
        return ("linear", linear, None)
    kv = _match_kv_update(node, dynamic)
    if kv is not None and _same_float_dtype(node, *kv[1:]):
        return (kv[0], tuple(kv[1:]), None)
    silu = _match_silu_mul(node, dynamic)
    if silu is not None and _same_float_dtype(node, silu[0], silu[1]):
        return ("silu_mul", silu, None)
    return None


def _tag_fits(node: LazyNode, tag) -> bool:
    kind, inputs, argument = tag
    if kind == "rms_norm":
        x, w = inputs
        return (_same_float_dtype(node, x, w) and len(w.shape) == 1 and x.shape
                and x.shape[-1] == w.shape[0] and x.shape == node.shape)
    if kind == "rope":
        x = inputs[0]
        if not (_same_float_dtype(node, x) and len(x.shape) == 4 and x.shape == node.shape):
            return False
        head = int(argument[0])
        if x.shape[-1] != head or head % 2:
            return False
        if len(inputs) == 2:
            position = inputs[1]
            if position.dtype != np.int32:
                return False
            if position.shape not in ((), (x.shape[0],)):
                return False
        return True
    if kind == "sdpa":
        q, k, v, mask = inputs
        if not _same_float_dtype(node, q, k, v):
            return False
        if len(q.shape) != 4 or len(k.shape) != 4 or k.shape != v.shape:
            return False
        b, h, t, hd = q.shape
        kb, kv, c, khd = k.shape
        if kb != b or khd != hd or h % kv or c > SDPA_MAX_KEYS or hd > 256:
            return False
        if not is_float(mask.dtype) or mask.dtype == np.float64 or len(mask.shape) > 4:
            return False
        try:
            return np.broadcast_shapes(mask.shape, (b, h, t, c)) == (b, h, t, c)
        except ValueError:
            return False
    if kind == "softmax":
        return _same_float_dtype(node, inputs[0])
    return False


# ---------------------------------------------------------------- emission
@dataclass
class PlannedProgram:
    steps: List[Step]
    storages: List[Storage]
    leaves: Tuple[LazyNode, ...]
    input_slots: Dict[LazyNode, int]
    output_specs: List[Tuple[str, object]]
    output_nodes: Tuple[LazyNode, ...]
    n_slots: int
    arena_bytes: int
    tape: np.ndarray
    source: str
    constants: List[object]
    signature: object


class Emitter:
    def __init__(self, compiler, plan: _HipGraphPlan, dynamic: Set[LazyNode],
                 donate: Set[LazyNode], specialized: bool):
        self.compiler = compiler
        self.plan = plan
        self.dynamic = dynamic
        self.donate = donate
        self.specialized = specialized
        self.steps: List[Step] = []
        self.values: Dict[LazyNode, PV] = {}
        self.storages: List[Storage] = []
        self.constants: List[object] = []
        self.leaf_storage: Dict[LazyNode, Storage] = {}
        self.rope_length = 1

    # -- buffers ------------------------------------------------------------
    def new_storage(self, kind: str, nbytes: int, **kw) -> Storage:
        storage = Storage(kind if nbytes > 0 else "empty", nbytes, **kw)
        self.storages.append(storage)
        return storage

    def new_value(self, shape, dtype, label="") -> PV:
        dtype = np.dtype(dtype)
        nbytes = _prod(shape) * dtype.itemsize
        storage = self.new_storage("arena", nbytes, label=label)
        return PV(shape, dtype, contiguous_strides(shape), storage)

    def constant(self, host: np.ndarray, label: str) -> PV:
        native = self.compiler.device.array(host)
        self.constants.append(native)
        storage = self.new_storage("const", host.nbytes, native=native, label=label)
        return PV(host.shape, host.dtype, contiguous_strides(host.shape), storage)

    def zeros(self, nbytes: int, label: str) -> PV:
        """A zero-filled device buffer owned by the program (kernel scratch
        such as self-resetting tickets)."""
        native = self.compiler.device.zeros((max(nbytes // 4, 1),), np.int32)
        self.constants.append(native)
        storage = self.new_storage("const", native.nbytes, native=native, label=label)
        return PV(native.shape, np.int32, (1,), storage)

    def add(self, kind: int, ins, outs, **attrs) -> Step:
        step = Step(kind, list(ins), list(outs), dict(attrs))
        self.steps.append(step)
        return step

    def copy_dense(self, pv: PV) -> PV:
        """A fresh contiguous, 256-byte aligned copy of ``pv``."""
        out = self.new_value(pv.shape, pv.dtype, "materialized")
        if out.size:
            self.add(K_COPY, [pv], [out])
        return out

    def materialize(self, pv: PV) -> PV:
        if pv.contiguous():
            return pv
        out = self.new_value(pv.shape, pv.dtype, "materialized")
        if out.size:
            self.add(K_COPY, [pv], [out])
        return out

    # -- driver -------------------------------------------------------------
    def run(self) -> None:
        nodes = self.plan.nodes()
        for node in nodes:
            if node.op is not None and op_of(node) is not Op.GATHER:
                if node.dtype == np.float64:
                    raise TypeError(
                        "the hip backend does not support float64; create this tensor as float32"
                    )
        self._scan_cache_lengths(nodes)
        for node in nodes:
            self.values[node] = self.emit(node)

    def _scan_cache_lengths(self, nodes) -> None:
        """RoPE tables must cover every position a program can see: the cache
        length of its attention and the sequence length of its rope nodes."""
        length = 1
        has_position = False
        for node in nodes:
            lowering = self.plan.lowering(node)
            if lowering is None:
                continue
            if lowering[0] == "sdpa":
                length = max(length, lowering[1][1].shape[2])
            if lowering[0] == "rope":
                x = lowering[1][0]
                length = max(length, x.shape[2] + int(lowering[2][2]))
                has_position = has_position or len(lowering[1]) == 2
        if has_position and length <= 1:
            length = 65536
        self.rope_length = length

    def emit(self, node: LazyNode) -> PV:
        if node.op is None:
            return self.emit_leaf(node)
        lowering = self.plan.lowering(node)
        if lowering is not None:
            kind, inputs, argument = lowering
            args = [self.values[parent] for parent in inputs]
            handler = getattr(self, "lower_" + kind)
            return handler(node, args, argument)
        args = [self.values[parent] for parent in node.inputs]
        handler = getattr(self, "op_" + op_of(node).name.lower())
        return handler(node, args)

    def emit_leaf(self, node: LazyNode) -> PV:
        dtype = node.dtype
        if dtype == np.float64:
            raise TypeError("the hip backend does not support float64; create this tensor as float32")
        dtype_code(dtype)  # raises TypeError for unsupported dtypes
        nbytes = _prod(node.shape) * dtype.itemsize
        if self.specialized and node not in self.dynamic:
            native = self.compiler._load_input(node)
            self.constants.append(native)
            storage = self.new_storage("const", nbytes, leaf=node, native=native, label="captured")
        else:
            storage = self.new_storage("input", nbytes, leaf=node, label="input")
        self.leaf_storage[node] = storage
        return PV(node.shape, dtype, contiguous_strides(node.shape), storage)

    # -- the six ops ------------------------------------------------------------
    def op_reshape(self, node, args):
        source = args[0]
        if source.contiguous():
            return PV(node.shape, node.dtype, contiguous_strides(node.shape), source.storage, source.offset)
        dense = self.materialize(source)
        return PV(node.shape, node.dtype, contiguous_strides(node.shape), dense.storage, dense.offset)

    def op_permute(self, node, args):
        source = args[0]
        order = tuple(node.arg)
        return PV(node.shape, node.dtype, tuple(source.strides[a] for a in order),
                  source.storage, source.offset)

    def op_elementwise(self, node, args):
        expression = (str(node.arg), node.dtype.str) + tuple(("input", i) for i in range(len(args)))
        return self.elementwise(node, args, expression)

    def lower_elementwise_fusion(self, node, args, expression):
        return self.elementwise(node, args, expression)

    def elementwise(self, node, args, expression) -> PV:
        if not is_float(node.dtype):
            raise PlanError(f"hip: elementwise {node.arg!r} with integer result {node.dtype} is not supported")
        if len(node.shape) > MAX_DIMS:
            raise PlanError("hip: elementwise rank above 8")
        out = self.new_value(node.shape, node.dtype, "elementwise")
        if out.size == 0:
            return out
        ops: List[int] = []

        def visit(term) -> int:
            if term[0] == "input":
                return int(term[1])
            registers = [visit(child) for child in term[2:]]
            code = OPCODES[term[0]]
            a = registers[0]
            b = registers[1] if len(registers) > 1 else 0
            ops.append(code | (a << 8) | (b << 16) | (dtype_code(np.dtype(term[1])) << 24))
            return len(args) + len(ops) - 1

        # Registers of ops are numbered after the inputs; visit assigns them
        # in post-order, so operand registers always precede their op.
        visit(expression)
        if len(args) > MAX_EW_INPUTS or len(ops) > MAX_EW_OPS:
            raise PlanError("hip: fused elementwise chain too large")
        for pv in args:
            dtype_code(pv.dtype)
        self.add(K_ELEMENTWISE, args, [out], expression=expression, ops=ops)
        return out

    def op_reduce(self, node, args):
        kind, axes, keepdims = node.arg
        source = args[0]
        if not is_float(source.dtype):
            raise PlanError("hip: reductions over integer tensors are not supported")
        if len(source.shape) > MAX_DIMS:
            raise PlanError("hip: reduce rank above 8")
        out = self.new_value(node.shape, node.dtype, "reduce")
        reduced = [d for d in range(len(source.shape)) if d in axes]
        if _prod([source.shape[d] for d in reduced]) == 0:
            if kind == "max":
                raise ValueError("zero-size array to reduction operation maximum which has no identity")
            if out.size:
                self.add(K_FILL, [], [out], words=(out.size * out.itemsize + 3) // 4)
            return out
        if out.size == 0:
            return out
        self.add(K_REDUCE, [source], [out], reduction=kind, axes=tuple(axes))
        return out

    def op_matmul(self, node, args):
        a, b = args
        if self._is_placement(a, b, node):
            # A @ eye(S, C): A's columns in the first S output columns, zeros
            # after them (the prefill KV-cache placement, llama.py
            # LlamaForCausalLM.prefill: (K^T @ eye(S, C))^T).  The result is
            # stored with its last two axes swapped -- the (C, D) layout of
            # the cache the graph transposes it back into -- so that
            # transpose is a view and the placement one row-contiguous copy.
            shape = tuple(node.shape)
            swapped = shape[:-2] + (shape[-1], shape[-2])
            dense = self.new_value(swapped, node.dtype, "placement")
            strides = dense.strides[:-2] + (dense.strides[-1], dense.strides[-2])
            out = PV(shape, node.dtype, strides, dense.storage, dense.offset)
            if a.shape[-1] != shape[-1]:  # columns past S: zeros (S == C: the copy covers all)
                self.add(K_FILL, [], [dense], words=(dense.size * dense.itemsize + 3) // 4)
            view = PV(a.shape, node.dtype, strides, dense.storage, dense.offset)
            self.add(K_COPY, [a], [view])
            return out
        row = self._one_hot_row(a, b, node)
        if row is not None:
            # e_s^T @ B: row s of B (the prefill's last-position selector,
            # llama.py LlamaForCausalLM._forward): a copy of that row
            view = PV(tuple(node.shape), node.dtype, b.strides, b.storage, b.offset + row * b.strides[-2])
            out = self.new_value(node.shape, node.dtype, "selected_row")
            self.add(K_COPY, [view], [out])
            return out
        return self.matmul(node, a, b)

    @staticmethod
    def _one_hot_row(a: PV, b: PV, node) -> Optional[int]:
        """a is a captured constant (1, S) row holding a single 1 and zeros, b
        is (..., S, D) of the same dtype: then a @ b is row s of b.  (As for
        the placement, only for finite B does this equal the float product.)"""
        if len(a.shape) != 2 or a.shape[0] != 1 or a.storage.kind != "const" or len(b.shape) < 2:
            return None
        if not (a.dtype == b.dtype == node.dtype) or a.shape[1] != b.shape[-2]:
            return None
        if tuple(node.shape) != tuple(b.shape[:-2]) + (1, b.shape[-1]):
            return None
        leaf = getattr(a.storage, "leaf", None)
        if leaf is None or leaf.value is None:
            return None
        value = np.asarray(leaf.value)
        if value.dtype == BFLOAT16:
            from .dtypes import bf16_to_float32
            value = bf16_to_float32(value)
        value = value.astype(np.float32).reshape(-1)
        if value.size != a.shape[1]:
            return None
        hot = np.flatnonzero(value)
        if hot.size != 1 or value[hot[0]] != 1.0:
            return None
        return int(hot[0])

    @staticmethod
    def _is_placement(a: PV, b: PV, node) -> bool:
        """b is a captured constant equal to eye(S, C), S <= C, and the
        product keeps A's dtype: then A @ b copies A into the first S
        columns.  (Only for finite A does this equal the float product: an
        inf in A would have spread NaN through its row.)"""
        if len(b.shape) != 2 or b.storage.kind != "const" or b.offset or not b.contiguous():
            return False
        if not (a.dtype == b.dtype == node.dtype) or len(a.shape) < 2 or len(node.shape) != len(a.shape):
            return False
        S, C = b.shape
        if a.shape[-1] != S or S > C or tuple(node.shape[:-1]) != tuple(a.shape[:-1]):
            return False
        leaf = getattr(b.storage, "leaf", None)
        if leaf is None or leaf.value is None:
            return False
        value = np.asarray(leaf.value)
        if value.shape != (S, C):
            return False
        if value.dtype == BFLOAT16:
            from .dtypes import bf16_to_float32
            value = bf16_to_float32(value)
        return bool(np.array_equal(value.astype(np.float32), np.eye(S, C, dtype=np.float32)))

    def matmul(self, node, a: PV, b: PV) -> PV:
        out = self.new_value(node.shape, node.dtype, "matmul")
        if out.size == 0:
            return out
        K = a.shape[-1]
        if K == 0:
            self.add(K_FILL, [], [out], words=(out.size * out.itemsize + 3) // 4)
            return out
        batch = node.shape[:-2]
        dims = []
        for i, size in enumerate(batch):
            if size == 1:
                continue
            ai = i - (len(batch) - (len(a.shape) - 2))
            bi = i - (len(batch) - (len(b.shape) - 2))
            sa = a.strides[ai] if ai >= 0 and a.shape[ai] != 1 else 0
            sb = b.strides[bi] if bi >= 0 and b.shape[bi] != 1 else 0
            dims.append([size, sa, sb])
        merged: List[List[int]] = []
        for dim in dims:
            if merged and merged[-1][1] == dim[1] * dim[0] and merged[-1][2] == dim[2] * dim[0]:
                merged[-1] = [merged[-1][0] * dim[0], dim[1], dim[2]]
            else:
                merged.append(dim)
        if len(merged) > 4:
            raise PlanError("hip: matmul with more than 4 independent batch dimensions")
        self.add(K_MATMUL, [a, b], [out], batch=merged)
        return out

    def op_gather(self, node, args):
        table, ids = args
        if not is_integer(ids.dtype) or ids.dtype not in (np.dtype(np.int32), np.dtype(np.int64)):
            raise TypeError("gather indices must be int32 or int64 on the hip backend")
        out = self.new_value(node.shape, node.dtype, "gather")
        if out.size == 0:
            return out
        if table.shape[0] == 0:
            raise IndexError("cannot gather from an empty table")
        table = self.materialize(table)
        ids = self.materialize(ids)
        if ids.size > 65535:
            raise PlanError("hip: gather of more than 65535 rows")
        self.add(K_GATHER, [table, ids], [out])
        return out

    # -- lowerings ----------------------------------------------------------------
    def lower_linear(self, node, args, _):
        x, w = args
        transposed = PV((w.shape[1], w.shape[0]), w.dtype, (w.strides[1], w.strides[0]), w.storage, w.offset)
        rows = _prod(x.shape[:-1])
        K = x.shape[-1]
        vector = 16 // x.itemsize if x.itemsize in (2, 4) else 0
        fits = (
            x.dtype == w.dtype == node.dtype and is_float(x.dtype)
            and 1 <= rows <= GEMV_MAX_ROWS and vector and K % vector == 0
            and w.contiguous() and (w.offset * w.itemsize) % 16 == 0
            and x.row_stride() is not None
        )
        if not fits:
            gemm = (
                x.dtype == w.dtype == node.dtype and is_float(x.dtype) and x.itemsize == 2
                and K % 8 == 0 and w.contiguous() and (w.offset * w.itemsize) % 16 == 0
                and rows > 0 and w.shape[0] > 0
            )
            if not gemm:
                return self.matmul(node, x, transposed)
            stride = x.row_stride()
            if stride is None or stride % 8 or (x.offset * x.itemsize) % 16:
                x = self.copy_dense(x)
            out = self.new_value(node.shape, node.dtype, "linear")
            self.add(K_GEMM, [x, w], [out], rows=rows, K=K, N=w.shape[0])
            return out
        out = self.new_value(node.shape, node.dtype, "linear")
        stage = rows * K * x.itemsize <= GEMV_STAGE_BYTES
        if not stage and (x.row_stride() % vector or (x.offset * x.itemsize) % 16):
            x = self.materialize(x)
        # The few positions of one sequence (x of shape (1, T, K), 2 <= T <= 8:
        # a verification block) are computed row-exactly: each row with the
        # arithmetic the single-token decode step uses, so a verified token
        # is the one greedy decoding would produce.  Batches of independent
        # sequences ((B, 1, K)) take the MFMA kernel unless
        # choose_batch_row_exact moves them (after sibling merging).
        exact = (x.itemsize == 2 and len(x.shape) == 3 and x.shape[0] == 1
                 and 2 <= x.shape[1] <= 8 and rows == x.shape[1])
        self.add(K_GEMV, [x], [out], segments=[{"w": w, "out": out, "res": None}],
                 prologue=None, silu=False, rows=rows, K=K, exact=exact)
        return out

    def lower_rms_norm(self, node, args, eps):
        x, w = args
        if x.row_stride() is None:
            x = self.materialize(x)
        out = self.new_value(node.shape, node.dtype, "rms_norm")
        if out.size:
            self.add(K_RMSNORM, [x, w], [out], eps=float(eps))
        return out

    def lower_rope(self, node, args, argument):
        head, theta, offset = int(argument[0]), float(argument[1]), int(argument[2])
        x = args[0]
        position = args[1] if len(args) == 2 else None
        out = self.new_value(node.shape, node.dtype, "rope")
        table = self.compiler._rope_table(head, theta, node.dtype, self.rope_length)
        self.constants.append(table)
        table_pv = PV(table.shape, table.dtype, contiguous_strides(table.shape),
                      self._const_storage(table, "rope_table"))
        mode = 0 if position is None else (1 if position.shape == () else 2)
        self.add(K_ROPE, [x, position, table_pv], [out], mode=mode, offset=offset,
                 table_length=int(table.shape[0]))
        return out

    def _const_storage(self, native, label) -> Storage:
        for storage in self.storages:
            if storage.kind == "const" and storage.native is native:
                return storage
        return self.new_storage("const", native.nbytes, native=native, label=label)

    def lower_sdpa(self, node, args, scale):
        q, k, v, mask = args
        # (B, H, T, hd) stored as (B, T, H, hd): the graph transposes the
        # heads back next to each other before o_proj, which is then a view
        B, H, T, hd = node.shape
        dense = self.new_value((B, T, H, hd), node.dtype, "sdpa")
        out = PV(tuple(node.shape), node.dtype, (T * H * hd, hd, H * hd, 1), dense.storage, dense.offset)
        if out.size:
            causal = self._causal_mask_value(mask, q.shape[2], k.shape[2], q.dtype)
            self.add(K_SDPA, [q, k, v, mask], [out], divisor=float(1.0 / float(scale)),
                     causal=causal)
        return out

    @staticmethod
    def _causal_mask_value(mask: Optional[PV], T: int, C: int, dtype) -> Optional[float]:
        """The value above the diagonal if ``mask`` is a captured constant
        whose every (T, C) slice, read through the view's shape, strides and
        offset, is exactly the causal triangle (0 on and below the diagonal,
        one value <= -1e4 above it) for T == C, else None.  Reading through
        the view matters: a transposed triangle (anti-causal) is a view of
        the same storage with other strides."""
        if mask is None or T != C or T < 2 or mask.storage.kind != "const":
            return None
        leaf = getattr(mask.storage, "leaf", None)
        if leaf is None or leaf.value is None or np.dtype(mask.dtype) != np.dtype(dtype):
            return None
        if len(mask.shape) < 2 or tuple(mask.shape[-2:]) != (T, C):
            return None
        flat = np.asarray(leaf.value).reshape(-1)
        index = mask.offset + sum(
            np.arange(size).reshape((1,) * axis + (size,) + (1,) * (len(mask.shape) - axis - 1)) * stride
            for axis, (size, stride) in enumerate(zip(mask.shape, mask.strides)))
        index = np.broadcast_to(index, mask.shape)
        if index.size == 0 or index.min() < 0 or index.max() >= flat.size:
            return None
        grids = flat[index].reshape(-1, T, C)
        if grids.dtype == BFLOAT16:
            from .dtypes import bf16_to_float32
            grids = bf16_to_float32(grids)
        grids = grids.astype(np.float32)
        above = grids[:, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]]
        lower = np.tril(np.ones((T, C), bool))
        if not np.all(grids[:, lower] == 0) or above.size == 0 or not np.all(above == above.flat[0]):
            return None
        return float(above.flat[0]) if above.flat[0] <= -1e4 + 16 else None

    def lower_softmax(self, node, args, axis):
        source = args[0]
        out = self.new_value(node.shape, node.dtype, "softmax")
        if out.size:
            self.add(K_SOFTMAX, [source], [out], axis=int(axis))
        return out

    def _in_place_ok(self, cache_node: LazyNode, cache: PV) -> bool:
        return (cache_node in self.donate and cache.storage.kind == "input"
                and cache.whole())

    def lower_kv_write(self, node, args, _):
        cache, x, w = args
        cache_node = self.plan.inputs(node)[0]
        if self._in_place_ok(cache_node, cache):
            out = PV(cache.shape, cache.dtype, cache.strides, cache.storage, cache.offset)
            self.add(K_KV_WRITE, [cache, x, w], [out], in_place=True, donated=cache_node)
            return out
        out = self.new_value(node.shape, node.dtype, "kv_cache")
        self.add(K_KV_WRITE, [cache, x, w], [out], in_place=False)
        return out

    def lower_kv_place(self, node, args, _):
        cache, x, placement, w = args
        cache_node = self.plan.inputs(node)[0]
        if self._in_place_ok(cache_node, cache):
            out = PV(cache.shape, cache.dtype, cache.strides, cache.storage, cache.offset)
            self.add(K_KV_PLACE, [cache, x, placement, w], [out], in_place=True, donated=cache_node)
            return out
        out = self.new_value(node.shape, node.dtype, "kv_cache")
        self.add(K_KV_PLACE, [cache, x, placement, w], [out], in_place=False)
        return out

    def lower_silu_mul(self, node, args, _):
        g, u, one = args
        expression = ("mul", node.dtype.str,
                      ("div", node.dtype.str, ("input", 0),
                       ("add", node.dtype.str,
                        ("exp", node.dtype.str, ("neg", node.dtype.str, ("input", 0))),
                        ("input", 2))),
                      ("input", 1))
        out = self.elementwise(node, [g, u, one], expression)
        self.steps[-1].attrs["silu_mul"] = True
        return out


# ---------------------------------------------------------------- fusion passes
def _consumers(steps: List[Step], outputs: List[PV]) -> Dict[int, int]:
    counts: Dict[int, int] = {}
    for step in steps:
        seen = set()
        for pv in step.reads():
            key = id(pv.storage)
            if key not in seen:
                counts[key] = counts.get(key, 0) + 1
                seen.add(key)
    for pv in outputs:
        counts[id(pv.storage)] = counts.get(id(pv.storage), 0) + 1
    return counts


def _producer(steps: List[Step]) -> Dict[int, Tuple[int, Step]]:
    result = {}
    for index, step in enumerate(steps):
        for pv in step.outs:
            result[id(pv.storage)] = (index, step)
    return result


def mfma_gemv(step: Step) -> bool:
    """A GEMV the library runs on MFMA (2..16 rows of a 16-bit type, K a
    multiple of 32, every segment a whole number of 16-column tiles).  With
    an RMSNorm prologue it keeps the whole K in one block (no split over
    blocks)."""
    x = step.ins[0]
    return (2 <= step.attrs["rows"] <= 16 and x.itemsize == 2 and step.attrs["K"] % 32 == 0
            and not step.attrs.get("exact")
            and all(seg["w"].shape[0] % 16 == 0 for seg in step.attrs["segments"]))


GEMV_MFMA_BLOCKS = int(os.environ.get("CHOMIK_HIP_GEMV_MFMA_BLOCKS", "512"))
GEMV_MFMA_BLOCK_KSTEPS = int(os.environ.get("CHOMIK_HIP_GEMV_MFMA_BLOCK_KSTEPS", "64"))


def mfma_gemv_blocks(step: Step) -> int:
    """Blocks that share one 16-column tile of an MFMA GEMV, each over an
    equal share of K: doubled while the launch has fewer than
    GEMV_MFMA_BLOCKS blocks and each block keeps at least
    GEMV_MFMA_BLOCK_KSTEPS k-steps of 32.  Narrow matrices over a long K
    (2048 columns over K = 8192: 17.4 -> 13.9 us at batch 8) otherwise occupy
    only half of the CUs; below 64 k-steps per block (K = 2048 split four
    ways) the partial exchange costs more than the CUs gain."""
    if not mfma_gemv(step) or step.attrs["prologue"] is not None:
        return 1
    segments = step.attrs["segments"]
    cols = segments[0]["w"].shape[0] if step.attrs["silu"] else sum(seg["w"].shape[0] for seg in segments)
    tiles, ksteps = cols // 16, step.attrs["K"] // 32
    kb = 1
    while (tiles * kb < GEMV_MFMA_BLOCKS and ksteps % (kb * 8) == 0
           and ksteps // (kb * 2) >= max(16, GEMV_MFMA_BLOCK_KSTEPS)):
        kb *= 2
    return kb


def _gemv_tiles(step: Step) -> int:
    segments = step.attrs["segments"]
    cols = segments[0]["w"].shape[0] if step.attrs["silu"] else sum(seg["w"].shape[0] for seg in segments)
    return cols // 16


def gemv_partial_bytes(step: Step, kb: int) -> int:
    """Partial tiles of a split MFMA GEMV: kb 16x16 float32 tiles per column
    tile and B operand."""
    return _gemv_tiles(step) * kb * (2 if step.attrs["silu"] else 1) * 256 * 4


def attach_gemv_workspace(steps: List[Step], emitter: "Emitter") -> List[Step]:
    """Gives every MFMA GEMV split over blocks one shared, zero-initialised
    workspace (p[14]): a ticket region of one int32 per tile of the widest
    such GEMV (256-byte aligned, n[25] bytes, always back at zero after a
    launch: the tickets reset themselves), then the partial tiles of the
    largest.  Steps run in order, so one buffer serves all of them."""
    split = [(step, mfma_gemv_blocks(step)) for step in steps if step.kind == K_GEMV]
    split = [(step, kb) for step, kb in split if kb > 1]
    if not split:
        return steps
    ticket_bytes = -(-max(_gemv_tiles(step) for step, _ in split) * 4 // 256) * 256
    partial_bytes = max(gemv_partial_bytes(step, kb) for step, kb in split)
    workspace = emitter.zeros(ticket_bytes + partial_bytes, "gemv_workspace")
    for step, kb in split:
        step.attrs.update(blocks=kb, workspace=workspace, ticket_bytes=ticket_bytes)
    return steps


def fuse_rmsnorm_prologue(steps: List[Step], outputs: List[PV]) -> List[Step]:
    counts = _consumers(steps, outputs)
    removed = set()
    for index, step in enumerate(steps):
        if step.kind != K_RMSNORM:
            continue
        normed = step.outs[0]
        users = [s for s in steps if any(pv.storage is normed.storage for pv in s.reads())]
        if not users or counts.get(id(normed.storage), 0) != len(users):
            continue
        x, w = step.ins
        ok = all(
            u.kind == K_GEMV and u.attrs["prologue"] is None and u.ins[0].same_data(normed)
            and u.attrs["rows"] * u.attrs["K"] * normed.itemsize <= GEMV_STAGE_BYTES
            and (not mfma_gemv(u) or w.dtype == x.dtype)
            and x.row_stride() is not None
            for u in users
        )
        if not ok:
            continue
        for u in users:
            u.attrs["prologue"] = {"x": x, "w": w, "eps": step.attrs["eps"]}
            u.ins = [x, w]
        removed.add(id(step))
    return [s for s in steps if id(s) not in removed]


def fuse_silu_gemv(steps: List[Step], outputs: List[PV]) -> List[Step]:
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    for step in steps:
        if step.kind != K_ELEMENTWISE or not step.attrs.get("silu_mul"):
            continue
        g, u = step.ins[0], step.ins[1]
        pg = producer.get(id(g.storage))
        pu = producer.get(id(u.storage))
        if not pg or not pu:
            continue
        gs, us = pg[1], pu[1]
        if gs.kind != K_GEMV or us.kind != K_GEMV or gs is us:
            continue
        if len(gs.attrs["segments"]) != 1 or len(us.attrs["segments"]) != 1:
            continue
        if counts.get(id(g.storage)) != 1 or counts.get(id(u.storage)) != 1:
            continue
        if not (g.whole() and u.whole()):
            continue
        same_input = gs.ins[0].same_data(us.ins[0]) if gs.attrs["prologue"] is None else (
            us.attrs["prologue"] is not None
            and gs.attrs["prologue"]["x"].same_data(us.attrs["prologue"]["x"])
            and gs.attrs["prologue"]["w"].storage is us.attrs["prologue"]["w"].storage)
        if not same_input or (gs.attrs["prologue"] is None) != (us.attrs["prologue"] is None):
            continue
        out = step.outs[0]
        gs.attrs["segments"] = [
            {"w": gs.attrs["segments"][0]["w"], "out": out, "res": None},
            {"w": us.attrs["segments"][0]["w"], "out": out, "res": None},
        ]
        gs.attrs["silu"] = True
        gs.outs = [out]
        removed.add(id(us))
        removed.add(id(step))
    return [s for s in steps if id(s) not in removed]


def fuse_residual(steps: List[Step], outputs: List[PV]) -> List[Step]:
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    for step in steps:
        if step.kind != K_ELEMENTWISE or step.attrs.get("silu_mul"):
            continue
        expression = step.attrs["expression"]
        if not (expression[0] == "add" and len(expression) == 4
                and expression[2][0] == "input" and expression[3][0] == "input"
                and len(step.ins) == 2):
            continue
        out = step.outs[0]
        for y_index in (1, 0):
            y, h = step.ins[y_index], step.ins[1 - y_index]
            found = producer.get(id(y.storage))
            if not found:
                continue
            gemv_index, gemv = found
            if gemv.kind != K_GEMV or gemv.attrs["silu"] or id(gemv) in removed:
                continue
            h_producer = producer.get(id(h.storage))
            if h_producer is not None and h_producer[0] >= gemv_index:
                continue  # the residual is computed after the GEMV runs
            segments = [s for s in gemv.attrs["segments"] if s["out"].storage is y.storage]
            if len(segments) != 1 or segments[0]["res"] is not None:
                continue
            if counts.get(id(y.storage)) != 1 or not y.whole():
                continue
            if h.shape != out.shape or not h.contiguous() or h.dtype != out.dtype:
                continue
            if _prod(y.shape) != _prod(out.shape) or y.dtype != out.dtype:
                continue
            segments[0]["res"] = h
            segments[0]["out"] = out
            gemv.outs = [s["out"] for s in gemv.attrs["segments"]]
            gemv.ins = gemv.ins + [h]
            removed.add(id(step))
            break
    return [s for s in steps if id(s) not in removed]


def fuse_gemm_epilogues(steps: List[Step], outputs: List[PV]) -> List[Step]:
    """Prefill: ``silu(g) * u`` of two GEMMs over the same input -> one GEMM
    with both weights and the SiLU epilogue; ``h + y`` of a GEMM output ->
    the GEMM's residual epilogue (the GEMV fusions, for many rows)."""
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    for step in steps:
        if step.kind != K_ELEMENTWISE or not step.attrs.get("silu_mul"):
            continue
        g, u = step.ins[0], step.ins[1]
        pg, pu = producer.get(id(g.storage)), producer.get(id(u.storage))
        if not pg or not pu:
            continue
        gs, us = pg[1], pu[1]
        if gs.kind != K_GEMM or us.kind != K_GEMM or gs is us or gs.attrs.get("res") or us.attrs.get("res"):
            continue
        if not gs.ins[0].same_data(us.ins[0]) or gs.attrs["N"] != us.attrs["N"] or gs.attrs["K"] != us.attrs["K"]:
            continue
        if counts.get(id(g.storage)) != 1 or counts.get(id(u.storage)) != 1 or not (g.whole() and u.whole()):
            continue
        out = step.outs[0]
        if not out.whole() or _prod(out.shape) != gs.attrs["rows"] * gs.attrs["N"]:
            continue
        gs.attrs["up"] = us.ins[1]
        gs.ins = [gs.ins[0], gs.ins[1], us.ins[1]]
        gs.outs = [out]
        removed.update({id(us), id(step)})
    steps = [s for s in steps if id(s) not in removed]
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    for step in steps:
        if step.kind != K_ELEMENTWISE or step.attrs.get("silu_mul"):
            continue
        expression = step.attrs["expression"]
        if not (expression[0] == "add" and len(expression) == 4 and expression[2][0] == "input"
                and expression[3][0] == "input" and len(step.ins) == 2):
            continue
        out = step.outs[0]
        for y_index in (1, 0):
            y, h = step.ins[y_index], step.ins[1 - y_index]
            found = producer.get(id(y.storage))
            if not found:
                continue
            gemm_index, gemm = found
            if gemm.kind != K_GEMM or gemm.attrs.get("up") is not None or gemm.attrs.get("res") is not None:
                continue
            h_producer = producer.get(id(h.storage))
            if h_producer is not None and h_producer[0] >= gemm_index:
                continue
            if counts.get(id(y.storage)) != 1 or not y.whole() or not out.whole():
                continue
            if h.shape != out.shape or not h.contiguous() or h.dtype != out.dtype or y.dtype != out.dtype:
                continue
            if _prod(out.shape) != gemm.attrs["rows"] * gemm.attrs["N"] or h.offset % 8:
                continue
            gemm.attrs["res"] = h
            gemm.ins = gemm.ins + [h]
            gemm.outs = [out]
            removed.add(id(step))
            break
    return [s for s in steps if id(s) not in removed]


def decode_attention_rows(itemsize: int) -> int:
    """Cache rows one pass of the decode-attention workgroup covers: 256
    threads, one 16-byte vector per lane, 64-element rows."""
    return 256 // (64 * itemsize // 16)


def decode_attention_passes(B: int, KV: int, C: int, itemsize: int) -> int:
    """Passes (rows per workgroup / rows per pass) for the chunk kernel of
    the split-context decode attention: the most rows per workgroup that
    still leaves >= 1024 workgroups, else one pass (short caches: as many
    workgroups as rows allow, so the per-workgroup latency chain stays
    short)."""
    rows = decode_attention_rows(itemsize)
    if DECODE_ATTN_PASSES > 0:
        chosen = DECODE_ATTN_PASSES
    else:
        chosen = 1
        for passes in (4, 2):
            if B * KV * -(-C // (rows * passes)) >= 1024:
                chosen = passes
                break
    # the combining workgroup merges at most 64 chunks per KV head
    while chosen < 4 and -(-C // (rows * chosen)) > DECODE_ATTN_MAX_CHUNKS:
        chosen *= 2
    return chosen


def decode_attention_plan(B: int, KV: int, C: int, G: int, itemsize: int, divisor: float = 8.0) -> Dict[str, int]:
    """Kernel choice for the fused decode attention: ``passes`` 1, 2 or 4 is
    the chunk kernel (``chunks`` workgroups per KV head); ``passes`` 0 is the
    streaming kernel, whose ``chunks`` workgroups per KV head each stream
    ``rows`` cache rows in tiles of ``unroll`` passes; ``passes`` 8 is the
    MFMA kernel, one workgroup per KV head whose waves hold ``rows`` blocks
    of 32 cache rows each.  ``rows`` is the kernel's n[29] in both cases."""
    rpp = decode_attention_rows(itemsize)
    pow2 = divisor > 0 and math.frexp(divisor)[0] == 0.5
    blocks = -(-C // DECODE_ATTN_MFMA_BLOCK)
    if (itemsize == 2 and pow2 and DECODE_ATTN_PASSES == -2
            and blocks <= DECODE_ATTN_MFMA_WAVES * DECODE_ATTN_MFMA_MAX_BLOCKS):
        per_wave = -(-blocks // DECODE_ATTN_MFMA_WAVES)
        return {"passes": 8, "chunks": 1, "rows": per_wave, "unroll": 0}
    stream = DECODE_ATTN_PASSES == -1
    if DECODE_ATTN_PASSES in (0, -2):  # -2 where the MFMA kernel does not apply: as 0
        biggest = -(-C // (rpp * 4))
        stream = B * KV * biggest > DECODE_ATTN_STREAM_ABOVE or biggest > DECODE_ATTN_MAX_CHUNKS
    # the streaming kernel multiplies by the reciprocal of the score divisor,
    # exact only for a power of two (the usual sqrt(64) = 8)
    stream = stream and pow2
    if not stream:
        passes = decode_attention_passes(B, KV, C, itemsize)
        return {"passes": passes, "chunks": -(-C // (rpp * passes)), "rows": 0, "unroll": 0}
    target = max(1, min(DECODE_ATTN_MAX_CHUNKS, -(-DECODE_ATTN_STREAM_WGS // (B * KV))))
    rows = -(-C // target)
    rows = -(-rows // rpp) * rpp
    unroll = DECODE_ATTN_STREAM_UNROLL
    return {"passes": 0, "chunks": -(-C // rows), "rows": rows, "unroll": unroll}


def fuse_decode_attention(steps: List[Step], outputs: List[PV], emitter: "Emitter") -> List[Step]:
    """rope(q), rope(k), kv_write(K), kv_write(V), sdpa -> one decode_attention
    step (single new token, head size 64)."""
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    tickets: Optional[PV] = None
    partials: Dict[int, PV] = {}
    for index, step in enumerate(steps):
        if step.kind != K_SDPA:
            continue
        q, K, V, mask = step.ins
        if q.shape[2] != 1 or q.shape[3] != 64:
            continue
        found = [producer.get(id(pv.storage)) for pv in (q, K, V)]
        if any(f is None for f in found):
            continue
        rq, wk, wv = (f[1] for f in found)
        if rq.kind != K_ROPE or wk.kind != K_KV_WRITE or wv.kind != K_KV_WRITE:
            continue
        if rq.attrs["mode"] not in (1, 2) or not q.whole() or counts.get(id(q.storage)) != 1:
            continue
        cache_k, xk, w = wk.ins
        cache_v, xv, w2 = wv.ins
        if not (K.same_data(wk.outs[0]) and V.same_data(wv.outs[0])):
            continue
        if w.storage is not w2.storage or w.offset != w2.offset or w.strides != w2.strides:
            continue
        if wk.attrs["in_place"] != wv.attrs["in_place"]:
            continue
        rk_found = producer.get(id(xk.storage))
        if rk_found is None:
            continue
        rk = rk_found[1]
        if (rk.kind != K_ROPE or not xk.whole() or counts.get(id(xk.storage)) != 1
                or rk.ins[1] is None or rk.ins[1].storage is not rq.ins[1].storage
                or rk.ins[2].storage is not rq.ins[2].storage or rk.attrs != rq.attrs):
            continue
        if xv.shape[2] != 1 or rk.ins[0].shape[2] != 1:
            continue
        B, H, _, _ = q.shape
        KV, C = cache_k.shape[1], cache_k.shape[2]
        if cache_k.shape != cache_v.shape or cache_k.strides != cache_v.strides:
            continue
        if cache_k.strides[2:] != (64, 1) or cache_v.strides[2:] != (64, 1):
            continue
        if w.dtype != q.dtype or mask.dtype != q.dtype or H // KV not in (1, 2, 4, 8):
            continue
        if tickets is None or tickets.size < B * KV:
            tickets = emitter.zeros(4 * max(B * KV, 64), "tickets")
        plan = decode_attention_plan(B, KV, C, H // KV, q.itemsize, float(step.attrs["divisor"]))
        chunks = plan["chunks"]
        if chunks > DECODE_ATTN_MAX_CHUNKS:
            continue
        floats = B * H * chunks * 66 if chunks > 1 else 1
        if floats not in partials:
            partials[floats] = emitter.zeros(4 * floats, "attention_partials")
        fused = Step(K_DECODE_ATTN,
                     [rq.ins[0], rk.ins[0], xv, rq.ins[1], rq.ins[2], cache_k, cache_v, w, mask, tickets,
                      partials[floats]],
                     [step.outs[0], wk.outs[0], wv.outs[0]],
                     {"in_place": wk.attrs["in_place"], "table_length": rq.attrs["table_length"],
                      "mode": rq.attrs["mode"], "divisor": step.attrs["divisor"], "passes": plan["passes"],
                      "stream_rows": plan["rows"], "unroll": plan["unroll"]})
        steps[index] = fused
        removed.update({id(rq), id(rk), id(wk), id(wv)})
    return [s for s in steps if id(s) not in removed]


def fuse_block_attention(steps: List[Step], outputs: List[PV], emitter: "Emitter") -> List[Step]:
    """rope(q) + sdpa of a verification block (T = 2..8 query rows of one
    sequence at positions p .. p + T - 1, head size 64, 16-bit) -> one
    read-only decode_attention step: the T rows run as T "sequences" over the
    one cache (batch stride 0), each with the decode step's own arithmetic
    (the chunk kernel, planned as for one sequence), so a block row equals the
    single-token step at its position.  The caches are written before by the
    block's own KV placement steps, which stay."""
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed = set()
    tickets: Optional[PV] = None
    partials: Dict[int, PV] = {}
    for index, step in enumerate(steps):
        if step.kind != K_SDPA:
            continue
        q, K, V, mask = step.ins
        Bq, H, T, hd = q.shape
        if Bq != 1 or not 2 <= T <= 8 or hd != 64 or q.itemsize != 2:
            continue
        found = producer.get(id(q.storage))
        if found is None:
            continue
        rq = found[1]
        if rq.kind != K_ROPE or rq.attrs["mode"] != 1 or rq.attrs["offset"] != 0:
            continue
        if not q.whole() or counts.get(id(q.storage)) != 1 or rq.ins[0].shape != q.shape:
            continue
        if len(K.shape) != 4 or K.shape[0] != 1 or K.shape != V.shape or K.strides != V.strides:
            continue
        KV, C = K.shape[1], K.shape[2]
        if K.strides[2:] != (64, 1) or C < T or H % KV or H // KV not in (1, 2, 4, 8):
            continue
        if mask is None or mask.dtype != q.dtype or K.dtype != q.dtype:
            continue
        plan = decode_attention_plan(1, KV, C, H // KV, q.itemsize, float(step.attrs["divisor"]))
        if plan["passes"] not in (1, 2, 4) or plan["chunks"] > DECODE_ATTN_MAX_CHUNKS:
            continue
        if tickets is None or tickets.size < T * KV:
            tickets = emitter.zeros(4 * max(T * KV, 64), "tickets")
        floats = T * H * plan["chunks"] * 66 if plan["chunks"] > 1 else 1
        if floats not in partials:
            partials[floats] = emitter.zeros(4 * floats, "attention_partials")
        steps[index] = Step(K_DECODE_ATTN,
                            [rq.ins[0], None, None, rq.ins[1], rq.ins[2], K, V, None, mask, tickets,
                             partials[floats]],
                            [step.outs[0]],
                            {"in_place": False, "table_length": rq.attrs["table_length"], "mode": 3,
                             "divisor": step.attrs["divisor"], "passes": plan["passes"], "stream_rows": 0,
                             "unroll": 0, "read_only": True})
        removed.add(id(rq))
    return [s for s in steps if id(s) not in removed]


def _same_view(a: PV, b: PV) -> bool:
    return (a.storage is b.storage and a.offset == b.offset and tuple(a.shape) == tuple(b.shape)
            and tuple(a.strides) == tuple(b.strides) and a.dtype == b.dtype)


def fuse_block_kv_place(steps: List[Step], outputs: List[PV]) -> List[Step]:
    """A layer's key and value placement (two kv_place steps with the same
    placement, write mask and cache geometry, the keys coming from a rope
    step read by nothing else) -> one paired kv_place step that rotates the
    keys on load: a verification block's three launches per layer become
    one.  The fused step takes the later placement's place in the order, and
    only if nothing in between reads the earlier one's cache."""
    counts = _consumers(steps, outputs)
    producer = _producer(steps)
    removed: Set[int] = set()
    places = [(i, st) for i, st in enumerate(steps) if st.kind == K_KV_PLACE]
    for index, pk in places:
        if id(pk) in removed or pk.attrs.get("pair"):
            continue
        cache, x, placement, w = pk.ins
        found = producer.get(id(x.storage))
        if found is None:
            continue
        rope = found[1]
        if (rope.kind != K_ROPE or rope.attrs["mode"] not in (0, 1) or counts.get(id(x.storage)) != 1
                or not x.whole() or x.shape != rope.ins[0].shape or cache.shape[3] % 2):
            continue
        for jndex, pv in places:
            if pv is pk or id(pv) in removed or pv.attrs.get("pair"):
                continue
            cache_v, xv, placement_v, w_v = pv.ins
            rope_v = producer.get(id(xv.storage))
            if rope_v is not None and rope_v[1].kind == K_ROPE:
                continue
            if not (_same_view(placement_v, placement) and _same_view(w_v, w)
                    and pv.attrs["in_place"] == pk.attrs["in_place"] and cache_v.shape == cache.shape
                    and cache_v.strides == cache.strides and cache_v.dtype == cache.dtype
                    and xv.shape == x.shape and xv.dtype == x.dtype):
                continue
            first, last = sorted((index, jndex))
            early = steps[first]
            between = steps[first + 1:last]
            if any(pv2.storage is early.outs[0].storage or pv2.storage is early.ins[0].storage
                   for st in between for pv2 in st.reads()):
                continue
            fused = Step(K_KV_PLACE, [cache, rope.ins[0], placement, w, cache_v, xv, rope.ins[2], rope.ins[1]],
                         [pk.outs[0], pv.outs[0]],
                         dict(pk.attrs, pair=True, rope={"mode": rope.attrs["mode"], "offset": rope.attrs["offset"],
                                                         "table_length": rope.attrs["table_length"]}))
            steps[last] = fused
            removed.update({id(early), id(rope)})
            break
    return [st for st in steps if id(st) not in removed]


def fuse_attention_projection(steps: List[Step], outputs: List[PV]) -> List[Step]:
    """Batch-1 chunk decode attention whose output feeds only the next
    single-row GEMV (the o projection, residual epilogue or none) -> the
    attention stores its per-chunk partials only and a K_ATTN_PROJ step
    combines them while its weight rows stream (the attention's own combine
    needs a cross-workgroup ticket and three memory round trips)."""
    if not ATTN_PROJ_FUSE:
        return steps
    counts = _consumers(steps, outputs)
    for index, att in enumerate(steps):
        if att.kind != K_DECODE_ATTN or att.attrs["passes"] not in (1, 2, 4) or att.attrs.get("read_only"):
            continue
        q, partials = att.ins[0], att.ins[10]
        out = att.outs[0]
        B, H = q.shape[0], q.shape[1]
        C = att.ins[5].shape[2]
        chunks = -(-C // (decode_attention_rows(q.itemsize) * att.attrs["passes"]))
        if B != 1 or q.itemsize != 2 or H * 64 not in (1024, 2048) or not 2 <= chunks <= ATTN_PROJ_MAX_CHUNKS:
            continue
        if not out.whole() or counts.get(id(out.storage)) != 1:
            continue
        users = [(i, s) for i, s in enumerate(steps) if any(pv.storage is out.storage for pv in s.reads())]
        if len(users) != 1:
            continue
        at, proj = users[0]
        if (proj.kind != K_GEMV or proj.attrs["silu"] or proj.attrs["prologue"] is not None
                or proj.attrs["rows"] != 1 or proj.attrs["K"] != H * 64 or len(proj.attrs["segments"]) != 1
                or proj.attrs.get("workspace") is not None or not proj.ins[0].same_data(out)):
            continue
        seg = proj.attrs["segments"][0]
        w, res, y = seg["w"], seg["res"], seg["out"]
        if not (w.contiguous() and w.dtype == q.dtype and (w.offset * w.itemsize) % 16 == 0
                and y.contiguous() and y.dtype == q.dtype
                and (res is None or (res.contiguous() and res.dtype == q.dtype))):
            continue
        att.attrs["partials_only"] = True
        steps[at] = Step(K_ATTN_PROJ, [partials, w, res], [y],
                         {"N": w.shape[0], "K": H * 64, "H": H, "chunks": chunks})
    return steps


GEMM_SEGMENT_WIDTH = 128  # segment widths of a merged GEMM: whole 128-column tiles


def merge_sibling_gemms(steps: List[Step]) -> List[Step]:
    """Plain GEMMs of the same A (the prefill q, k and v projections) -> one
    launch with up to four output segments: one pass over A, and the narrow
    k and v products (256 columns) no longer run as launches of their own."""
    removed = set()
    for i, first in enumerate(steps):
        if first.kind != K_GEMM or id(first) in removed or first.attrs.get("res") is not None \
                or first.attrs.get("up") is not None:
            continue
        group = [first]
        for later in steps[i + 1:]:
            if len(group) == 4:
                break
            if later.kind != K_GEMM or id(later) in removed or later.attrs.get("res") is not None \
                    or later.attrs.get("up") is not None:
                continue
            if later.attrs["K"] != first.attrs["K"] or later.attrs["rows"] != first.attrs["rows"]:
                continue
            if not later.ins[0].same_data(first.ins[0]) or later.ins[0].dtype != first.ins[0].dtype:
                continue
            group.append(later)
        widths = [s.attrs["N"] for s in group]
        if len(group) < 2 or any(w % GEMM_SEGMENT_WIDTH for w in widths):
            continue
        if any(s.outs[0].row_stride() is None or s.ins[1].strides[-1] != 1 for s in group):
            continue
        first.attrs["segments"] = [(s.ins[1], s.outs[0]) for s in group]
        first.attrs["N"] = sum(widths)
        first.ins = [first.ins[0]] + [s.ins[1] for s in group]
        first.outs = [s.outs[0] for s in group]
        removed.update(id(s) for s in group[1:])
    return [s for s in steps if id(s) not in removed]


def choose_batch_row_exact(steps: List[Step]) -> List[Step]:
    """Batch GEMVs (2..8 independent rows, 16-bit, K <= 2048) that run on
    the row-exact kernels, where those measured faster than the MFMA kernel
    (C4, batch 8, K = 2048): narrow launches (o_proj 2048x2048: 6.1 against
    7.5 us) and very tall ones (the 128256-row lm_head: 105 against
    112 us); the merged q/k/v (3072 rows: 13.8 against 10.2 us) and the
    gate/up pair (2 x 8192) stay on MFMA.  Decided on the merged launch, by
    the rows of all its segments."""
    if not GEMV_BATCH_ROW_EXACT:
        return steps
    for step in steps:
        a = step.attrs
        if step.kind != K_GEMV or a.get("exact"):
            continue
        x = a["prologue"]["x"] if a["prologue"] else step.ins[0]
        if x.itemsize != 2 or not 2 <= a["rows"] <= 8 or a["K"] > GEMV_BATCH_ROW_EXACT_MAX_K:
            continue
        n = sum(seg["w"].shape[0] for seg in a["segments"])
        if n <= 2048 or n >= 32768:
            a["exact"] = True
    return steps


def merge_sibling_gemvs(steps: List[Step]) -> List[Step]:
    removed = set()
    for i, first in enumerate(steps):
        if first.kind != K_GEMV or first.attrs["silu"] or id(first) in removed:
            continue
        for later in steps[i + 1:]:
            if len(first.attrs["segments"]) >= 4:
                break
            if later.kind != K_GEMV or later.attrs["silu"] or id(later) in removed:
                continue
            if later.attrs["rows"] != first.attrs["rows"] or later.attrs["K"] != first.attrs["K"]:
                continue
            if later.ins[0].dtype != first.ins[0].dtype:
                continue
            if not later.ins[0].same_data(first.ins[0]):
                continue
            p1, p2 = first.attrs["prologue"], later.attrs["prologue"]
            if (p1 is None) != (p2 is None):
                continue
            if p1 is not None and (p1["w"].storage is not p2["w"].storage or p1["eps"] != p2["eps"]
                                   or not p1["x"].same_data(p2["x"])):
                continue
            if any(s["res"] is not None for s in later.attrs["segments"]):
                # moving a residual read earlier is safe, but keep launches simple
                continue
            if len(first.attrs["segments"]) + len(later.attrs["segments"]) > 4:
                continue
            # The later GEMV moves up to ``first``: its weights are constants
            # and its input is ``first``'s, so nothing it reads is produced in
            # between.
            first.attrs["segments"].extend(later.attrs["segments"])
            first.outs = [s["out"] for s in first.attrs["segments"]]
            removed.add(id(later))
    return [s for s in steps if id(s) not in removed]


# ---------------------------------------------------------------- memory
def assign_memory(steps: List[Step], storages: List[Storage], outputs: List[PV]) -> int:
    for storage in storages:
        storage.first = storage.last = -1
    for index, step in enumerate(steps):
        for pv in step.outs:
            if pv.storage.first < 0:
                pv.storage.first = index
            pv.storage.last = max(pv.storage.last, index)
        for pv in step.reads():
            if pv.storage.first < 0:
                pv.storage.first = index
            pv.storage.last = max(pv.storage.last, index)
    for pv in outputs:
        pv.storage.last = len(steps)
    arena = [s for s in storages if s.kind == "arena" and s.first >= 0]
    arena.sort(key=lambda s: (-s.nbytes, s.first))
    placed: List[Storage] = []
    total = 0
    for storage in arena:
        size = (storage.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
        busy = sorted(
            (other.offset, other.offset + (other.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN)
            for other in placed
            if not (other.last < storage.first or storage.last < other.first)
        )
        offset = 0
        for begin, end in busy:
            if offset + size <= begin:
                break
            offset = max(offset, end)
        storage.offset = offset
        placed.append(storage)
        total = max(total, offset + size)
    return total


# ---------------------------------------------------------------- tape
def _ptr(pv: Optional[PV]) -> Tuple[int, int]:
    if pv is None or pv.storage.kind == "empty":
        return (-1, 0)
    storage = pv.storage
    base = storage.offset if storage.kind == "arena" else 0
    return (storage.slot, base + pv.offset * pv.itemsize)


def _pad(values: Sequence[int], length: int, fill: int = 0) -> List[int]:
    values = [int(v) for v in values]
    return values + [fill] * (length - len(values))


def _float_bits(value: float) -> int:
    return int(np.array([value], dtype=np.float32).view(np.uint32)[0])


def broadcast_strides(pv: PV, shape: Sequence[int]) -> List[int]:
    strides = [0] * len(shape)
    lead = len(shape) - len(pv.shape)
    for i, (size, stride) in enumerate(zip(pv.shape, pv.strides)):
        strides[lead + i] = 0 if size == 1 else stride
    return strides


def encode(step: Step) -> Tuple[int, List[Tuple[int, int]], List[int], List[float]]:
    kind = step.kind
    a = step.attrs
    if kind == K_FILL:
        out = step.outs[0]
        return kind, [_ptr(out)], [a["words"], 0], []
    if kind == K_COPY:
        src, dst = step.ins[0], step.outs[0]
        shape, src_strides, dst_strides = copy_order(src.shape, src.strides, dst.strides)
        strided = dst_strides != contiguous_strides(shape)
        return kind, [_ptr(src), _ptr(dst)], (
            [src.size, len(shape)] + _pad(shape, 8, 1) + _pad(src_strides, 8) + [src.itemsize]
            + [1 if strided else 0] + _pad(dst_strides if strided else (), 8)
        ), []
    if kind == K_ELEMENTWISE:
        out = step.outs[0]
        ins = step.ins
        ints = [out.size, len(out.shape)] + _pad(out.shape, 8, 1)
        ints += [len(ins), len(a["ops"]), dtype_code(out.dtype)]
        ints += _pad([dtype_code(pv.dtype) for pv in ins], 6)
        for k in range(6):
            ints += _pad(broadcast_strides(ins[k], out.shape), 8) if k < len(ins) else [0] * 8
        ints += _pad(a["ops"], 24)
        return kind, [_ptr(out)] + [_ptr(pv) for pv in ins], ints, []
    if kind == K_REDUCE:
        src, out = step.ins[0], step.outs[0]
        axes = a["axes"]
        kept = [d for d in range(len(src.shape)) if d not in axes]
        red = [d for d in range(len(src.shape)) if d in axes]
        ints = [out.size, _prod([src.shape[d] for d in red]), 0 if a["reduction"] == "sum" else 1,
                dtype_code(src.dtype), dtype_code(out.dtype), len(kept)]
        ints += _pad([src.shape[d] for d in kept], 8, 1) + _pad([src.strides[d] for d in kept], 8)
        ints += [len(red)] + _pad([src.shape[d] for d in red], 8, 1) + _pad([src.strides[d] for d in red], 8)
        return kind, [_ptr(src), _ptr(out)], ints, []
    if kind == K_GATHER:
        table, ids = step.ins
        out = step.outs[0]
        row_bytes = _prod(table.shape[1:]) * table.itemsize
        aligned16 = all((_ptr(pv)[1] % 16 == 0) for pv in (table, out))
        unit = 16 if row_bytes % 16 == 0 and aligned16 else (4 if row_bytes % 4 == 0 else 1)
        return kind, [_ptr(table), _ptr(ids), _ptr(out)], [
            ids.size, table.shape[0], row_bytes, dtype_code(ids.dtype), unit], []
    if kind == K_MATMUL:
        A, B = step.ins
        C = step.outs[0]
        batch = a["batch"]
        n_batch = _prod([d[0] for d in batch]) if batch else 1
        ints = [n_batch, A.shape[-2], B.shape[-1], A.shape[-1],
                dtype_code(A.dtype), dtype_code(B.dtype), dtype_code(C.dtype),
                A.strides[-2], A.strides[-1], B.strides[-2], B.strides[-1], len(batch)]
        ints += _pad([d[0] for d in batch], 4, 1) + _pad([d[1] for d in batch], 4) + _pad([d[2] for d in batch], 4)
        return kind, [_ptr(A), _ptr(B), _ptr(C)], ints, []
    if kind == K_SOFTMAX:
        src, out = step.ins[0], step.outs[0]
        axis = a["axis"]
        kept = [d for d in range(len(src.shape)) if d != axis]
        ints = [_prod([src.shape[d] for d in kept]), src.shape[axis], dtype_code(src.dtype),
                src.strides[axis], out.strides[axis], len(kept)]
        ints += _pad([src.shape[d] for d in kept], 8, 1) + _pad([src.strides[d] for d in kept], 8)
        ints += _pad([out.strides[d] for d in kept], 8)
        return kind, [_ptr(src), _ptr(out)], ints, []
    if kind == K_RMSNORM:
        x, w = step.ins
        out = step.outs[0]
        rows = _prod(x.shape[:-1])
        aligned = all(_ptr(pv)[1] % 16 == 0 for pv in (x, w, out))
        return kind, [_ptr(x), _ptr(w), _ptr(out)], [
            rows, x.shape[-1], x.row_stride(), dtype_code(x.dtype), dtype_code(w.dtype),
            1 if aligned else 0], [a["eps"]]
    if kind == K_ROPE:
        x, position, table = step.ins
        out = step.outs[0]
        # 16-byte aligned rows of x, the table and the output (vector kernel)
        aligned = (x.strides[3] == 1 and all(s % 8 == 0 for s in x.strides[:3])
                   and all(pv.offset % 8 == 0 for pv in (x, table, out)) and table.contiguous())
        return kind, [_ptr(x), _ptr(position), _ptr(table), _ptr(out)], (
            list(x.shape) + list(x.strides) + [dtype_code(x.dtype), a["mode"], a["offset"], a["table_length"],
                                               1 if aligned else 0]
        ), []
    if kind == K_SDPA:
        q, k, v, mask = step.ins
        out = step.outs[0]
        b, h, t, hd = q.shape
        c = k.shape[2]
        mask_strides = broadcast_strides(mask, (b, h, t, c))
        ints = [b, h, t, c, hd, k.shape[1], dtype_code(q.dtype)]
        ints += list(q.strides) + list(k.strides) + list(v.strides) + mask_strides + [dtype_code(mask.dtype)]
        causal = a.get("causal")
        aligned = all(pv.offset % 8 == 0 for pv in (q, k, v))
        ints += [1 if causal is not None else 0, 1 if aligned else 0]
        assert out.strides[3] == 1 or out.shape[3] == 1
        ints += list(out.strides[:3])
        return kind, [_ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(out)], ints, [
            a["divisor"], causal if causal is not None else 0.0]
    if kind == K_KV_WRITE:
        cache, x, w = step.ins
        out = step.outs[0]
        b, kv, c, hd = cache.shape
        xs = broadcast_strides(x, cache.shape)
        ws = broadcast_strides(w, (b, 1, c, 1))
        ints = [b, kv, c, hd, dtype_code(cache.dtype)] + xs + [ws[0], ws[2], 1 if a["in_place"] else 0]
        ints += list(cache.strides) + [dtype_code(w.dtype)]
        return kind, [_ptr(cache), _ptr(x), _ptr(w), _ptr(out)], ints, []
    if kind == K_KV_PLACE:
        cache, x, placement, w = step.ins[:4]
        out = step.outs[0]
        b, kv, c, hd = cache.shape
        t = x.shape[2]
        xs = broadcast_strides(x, (b, kv, t, hd))
        ws = broadcast_strides(w, (b, 1, c, 1))
        ints = [b, kv, c, hd, dtype_code(cache.dtype), t] + xs + list(placement.strides)
        ints += [ws[0], ws[2], 1 if a["in_place"] else 0] + list(cache.strides)
        ints += [dtype_code(placement.dtype), dtype_code(w.dtype)]
        ptrs = [_ptr(cache), _ptr(x), _ptr(placement), _ptr(w), _ptr(out)]
        if a.get("pair"):
            # the value placement (p[5..7]) and the keys' RoPE (table p[8],
            # position p[9])
            cache_v, xv, table, position = step.ins[4:8]
            ints += [1] + broadcast_strides(xv, (b, kv, t, hd))
            r = a["rope"]
            ints += [1, 1 if r["mode"] == 1 else 0, r["offset"], r["table_length"]]
            ptrs += [_ptr(cache_v), _ptr(xv), _ptr(step.outs[1]), _ptr(table), _ptr(position)]
        return kind, ptrs, ints, []
    if kind == K_DECODE_ATTN and a.get("read_only"):
        # T query rows of one block as T sequences over one cache (batch
        # stride 0): q strides (t, h, d), mask strides (t, h, c)
        q, _, _, position, table, cache_k, cache_v, _, mask, tickets, partials = step.ins
        out = step.outs[0]
        _, H, T, _ = q.shape
        KV, C = cache_k.shape[1], cache_k.shape[2]
        ms = broadcast_strides(mask, (1, H, T, C))
        ints = [T, H, KV, C, dtype_code(q.dtype), q.strides[2], q.strides[1], q.strides[3],
                0, 0, 0, 0, 0, 0, 3, a["table_length"], 0] + list(cache_k.strides[1:])
        ints += [0, 0, ms[2], ms[1], ms[3], dtype_code(mask.dtype), dtype_code(q.dtype),
                 0, a["passes"], 0, 0, 0, 1]
        ptrs = [_ptr(pv) for pv in (q, None, None, position, table, cache_k, cache_v, None, mask, out, None,
                                    None, tickets, partials)]
        return kind, ptrs, ints, [a["divisor"]]
    if kind == K_DECODE_ATTN:
        q, k, v, position, table, cache_k, cache_v, w, mask, tickets, partials = step.ins
        out, out_k, out_v = step.outs
        B, H = q.shape[0], q.shape[1]
        KV, C = cache_k.shape[1], cache_k.shape[2]
        ws = broadcast_strides(w, (B, 1, C, 1))
        ms = broadcast_strides(mask, (B, H, 1, C))
        ints = [B, H, KV, C, dtype_code(q.dtype),
                q.strides[0], q.strides[1], q.strides[3],
                k.strides[0], k.strides[1], k.strides[3],
                v.strides[0], v.strides[1], v.strides[3],
                a["mode"], a["table_length"]] + list(cache_k.strides)
        ints += [ws[0], ws[2], ms[0], ms[1], ms[3], dtype_code(mask.dtype), dtype_code(w.dtype),
                 1 if a["in_place"] else 0, a["passes"], a["stream_rows"], a["unroll"],
                 1 if a.get("partials_only") else 0, 0]
        ptrs = [_ptr(pv) for pv in (q, k, v, position, table, cache_k, cache_v, w, mask, out, out_k, out_v,
                                    tickets, partials)]
        return kind, ptrs, ints, [a["divisor"]]
    if kind == K_ATTN_PROJ:
        partials, w, res = step.ins
        ptrs = [_ptr(partials), _ptr(w), _ptr(res), _ptr(step.outs[0])]
        return kind, ptrs, [a["N"], a["K"], a["H"], a["chunks"], dtype_code(w.dtype)], []
    if kind == K_GEMM:
        x, w = step.ins[0], step.ins[1]
        out = step.outs[0]
        res, up = a.get("res"), a.get("up")
        segments = a.get("segments") or []  # [(w, out)] of merged siblings
        ptrs = [_ptr(x), _ptr(w), _ptr(out), _ptr(res), _ptr(up)]
        for sw, so in segments[1:]:
            ptrs += [_ptr(sw), _ptr(so)]
        ints = [a["rows"], a["N"], a["K"], dtype_code(x.dtype), x.row_stride(), w.strides[0],
                out.row_stride() if segments else a["N"],
                a["N"] if res is not None else 0, 1 if up is not None else 0,
                up.strides[0] if up is not None else 0, 1 if res is not None else 0]
        ints += [len(segments)] + _pad([sw.shape[0] for sw, _ in segments], 4)
        ints += _pad([so.row_stride() for _, so in segments], 4) + _pad([sw.strides[0] for sw, _ in segments], 4)
        return kind, ptrs, ints, []
    if kind == K_GEMV:
        segments = a["segments"]
        prologue = a["prologue"]
        x = prologue["x"] if prologue else step.ins[0]
        ptrs = [_ptr(x), _ptr(prologue["w"]) if prologue else (-1, 0)]
        ptrs += [_ptr(s["w"]) for s in segments] + [(-1, 0)] * (4 - len(segments))
        ptrs += [_ptr(s["out"]) for s in segments] + [(-1, 0)] * (4 - len(segments))
        ptrs += [_ptr(s["res"]) for s in segments] + [(-1, 0)] * (4 - len(segments))
        ptrs += [_ptr(a.get("workspace"))]
        rows, K = a["rows"], a["K"]
        n = [s["w"].shape[0] for s in segments]
        stage = rows * K * x.itemsize <= GEMV_STAGE_BYTES
        ints = [rows, K, x.row_stride(), dtype_code(x.dtype), len(segments),
                1 if prologue else 0, 1 if a["silu"] else 0]
        ints += _pad(n, 4)
        if a["silu"]:
            ints += _pad([n[0]], 4)
        else:
            ints += _pad(n, 4)
        ints += _pad([s["res"].shape[-1] if s["res"] is not None else 0 for s in segments], 4)
        vector = 16 // x.itemsize
        aligned = x.row_stride() % vector == 0 and (_ptr(x)[1] % 16) == 0
        ints += [dtype_code(prologue["w"].dtype) if prologue else 0, 1 if stage else 0, GEMV_SPLIT,
                 1 if aligned else 0, 0, a.get("blocks", 1), a.get("ticket_bytes", 0),
                 1 if a.get("exact") else 0, 0]
        return kind, ptrs, ints, [prologue["eps"] if prologue else 0.0]
    raise AssertionError(f"no encoder for step kind {kind}")


def copy_order(shape: Sequence[int], src_strides: Sequence[int], dst_strides: Sequence[int]):
    """The axes of an element copy in the order the kernel walks them: by
    destination stride, largest first (the last axis the destination's
    fastest), size-1 axes dropped and neighbours that are contiguous in both
    source and destination merged.  A transposed pair of views (the prefill
    KV placement) becomes a copy of contiguous rows."""
    axes = [d for d in range(len(shape)) if shape[d] != 1]
    axes.sort(key=lambda d: (-dst_strides[d], -src_strides[d]))
    dims = [[shape[d], src_strides[d], dst_strides[d]] for d in axes]
    merged: List[List[int]] = []
    for size, ss, ds in dims:
        if merged and merged[-1][1] == ss * size and merged[-1][2] == ds * size:
            merged[-1] = [merged[-1][0] * size, ss, ds]
        else:
            merged.append([size, ss, ds])
    if not merged:
        merged = [[1, 1, 1]]
    return (tuple(m[0] for m in merged), tuple(m[1] for m in merged), tuple(m[2] for m in merged))


def build_tape(steps: List[Step], n_slots: int, arena_bytes: int) -> np.ndarray:
    words = [0x43484950, 1, n_slots, len(steps), arena_bytes]
    for step in steps:
        kind, ptrs, ints, floats = encode(step)
        words += [kind, len(ptrs), len(ints), len(floats)]
        for slot, offset in ptrs:
            words += [slot, offset]
        words += [int(v) for v in ints]
        words += [_float_bits(v) for v in floats]
    return np.asarray(words, dtype=np.int64)


def describe(step: Step, names: Dict[int, str]) -> str:
    def name(pv: Optional[PV]) -> str:
        if pv is None:
            return "None"
        return names.setdefault(id(pv.storage), f"b{len(names)}")

    label = KIND_NAMES[step.kind]
    a = step.attrs
    if step.kind == K_GEMV:
        tags = []
        if a["prologue"]:
            tags.append("rms_norm")
        if a["silu"]:
            tags.append("silu_mul")
        if any(s["res"] is not None for s in a["segments"]):
            tags.append("residual")
        if a.get("exact"):
            tags.append("row_exact")
        label += f"[{'+'.join(tags)}]" if tags else ""
        weights = ", ".join(f"{name(s['w'])}{tuple(s['w'].shape)}" for s in a["segments"])
        x = a["prologue"]["x"] if a["prologue"] else step.ins[0]
        return (f"    {', '.join(name(o) for o in step.outs)} = {label}(x={name(x)}, "
                f"rows={a['rows']}, K={a['K']}, W=[{weights}])")
    if step.kind == K_ELEMENTWISE:
        label = "fused_elementwise" if len(a["ops"]) > 1 else f"elementwise_{a['expression'][0]}"
    if step.kind == K_DECODE_ATTN and a.get("read_only"):
        label = "decode_attention[block]"
    if step.kind == K_KV_PLACE and a.get("pair"):
        label = "kv_place[rope+pair]"
    ins = ", ".join(name(pv) for pv in step.ins)
    outs = ", ".join(name(pv) for pv in step.outs)
    shape = tuple(step.outs[0].shape) if step.outs else ()
    return f"    {outs} = {label}({ins})  # {shape} {dtype_name(step.outs[0].dtype) if step.outs else ''}"


# ---------------------------------------------------------------- driver
def plan_graph(compiler, outputs: Sequence[LazyNode], dynamic_inputs: Sequence[LazyNode],
               donate: Sequence[LazyNode] = ()) -> PlannedProgram:
    outputs = tuple(outputs)
    dynamic = set(dynamic_inputs)
    specialized = bool(dynamic_inputs)
    plan = choose_lowerings(outputs, dynamic)
    nodes = plan.nodes()
    leaves = tuple(node for node in nodes if node.op is None)
    emitter = Emitter(compiler, plan, dynamic, set(donate), specialized)
    emitter.run()
    out_pvs = [emitter.values[node] for node in outputs]

    steps = [s for s in emitter.steps if all(pv.storage.kind != "empty" for pv in s.outs)]
    steps = fuse_rmsnorm_prologue(steps, out_pvs)
    steps = fuse_silu_gemv(steps, out_pvs)
    steps = fuse_residual(steps, out_pvs)
    steps = fuse_gemm_epilogues(steps, out_pvs)
    steps = merge_sibling_gemvs(steps)
    steps = choose_batch_row_exact(steps)
    steps = merge_sibling_gemms(steps)
    steps = fuse_decode_attention(steps, out_pvs, emitter)
    steps = fuse_block_attention(steps, out_pvs, emitter)
    steps = fuse_block_kv_place(steps, out_pvs)
    steps = fuse_attention_projection(steps, out_pvs)
    steps = attach_gemv_workspace(steps, emitter)

    # Program outputs: leaves are returned as they are, whole intermediates
    # become caller-visible buffers, anything else is copied into one.
    specs: List[Tuple[str, object]] = []
    for node, pv in zip(outputs, out_pvs):
        storage = pv.storage
        if storage.kind == "empty":
            specs.append(("empty", node))
        elif storage.kind == "input" and pv.whole():
            specs.append(("input", storage.leaf))
        elif storage.kind == "const" and pv.whole():
            specs.append(("const", storage.native))
        elif storage.kind in ("arena", "output") and pv.whole():
            storage.kind = "output"
            specs.append(("output", storage))
        else:
            dense = emitter.new_storage("output", pv.size * pv.itemsize, label="output")
            target = PV(pv.shape, pv.dtype, contiguous_strides(pv.shape), dense)
            steps.append(Step(K_COPY, [pv], [target]))
            specs.append(("output", dense))
    arena_bytes = assign_memory(steps, emitter.storages, [])

    slot = 1
    input_slots: Dict[LazyNode, int] = {}
    for storage in emitter.storages:
        if storage.kind == "arena":
            storage.slot = 0
        elif storage.kind == "empty":
            storage.slot = -1
        elif storage.kind == "output" or storage.first >= 0:
            storage.slot = slot
            slot += 1
            if storage.kind == "input":
                input_slots[storage.leaf] = storage.slot
    tape = build_tape(steps, slot, arena_bytes)

    names: Dict[int, str] = {}
    lines = [f"# hip plan: {len(steps)} kernels, arena {arena_bytes} bytes"]
    lines += [describe(step, names) for step in steps]
    lines.append("    return (" + ", ".join(
        names.get(id(spec[1]), "input") if spec[0] == "output" else spec[0] for spec in specs) + ")")
    return PlannedProgram(
        steps=steps, storages=emitter.storages, leaves=leaves, input_slots=input_slots,
        output_specs=specs, output_nodes=outputs, n_slots=slot, arena_bytes=arena_bytes,
        tape=tape, source="\n".join(lines), constants=emitter.constants,
        signature=plan.signature(nodes),
    )
