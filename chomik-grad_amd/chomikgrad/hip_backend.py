"""The ``hip`` compiler plugin: MI355X (gfx950) execution of lazy graphs.

Implements the reference's plugin contract (chomikgrad/lazy.py:107-209):

* ``HIPDeviceAdapter``  -- ``DeviceAdapter`` (array, evaluate, synchronize,
  to_numpy, argmax, argmax_last_axis, dtype, load_safetensors, peak memory);
  the counterparts of CUDADeviceAdapter (cuda_backend.py:19-44) and
  MLXDeviceAdapter (mlx_backend.py:20-102).
* ``HIPProgram``        -- ``CompiledProgram.run(bindings, synchronize=False)``:
  binds inputs, queues the whole plan as one hipGraph launch and returns
  device arrays without waiting (CUDAProgram.run, cuda_backend.py:47-69).
* ``HIPCompiler``       -- ``Compiler.compile(outputs, dynamic_inputs)``:
  validates like the reference (empty outputs, non-leaf or foreign dynamic
  inputs raise ``ValueError``), captures non-dynamic leaves once (weights),
  accepts dynamic leaves of the portable or the lowered graph
  (mlx_backend.py:239-258) and caches unspecialised programs by structural
  signature (lazy.py:286-319).

The device work happens in ``libchomik_hip.so`` (include/chomik_hip.h),
reached through ctypes.  A missing library raises ``ImportError`` and a
missing GPU ``RuntimeError`` when the compiler is constructed; nothing ever
falls back to the host.
"""

from __future__ import annotations

import ctypes
import json
import mmap
import os
import struct
from pathlib import Path
from typing import Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np

from . import _hiplib
from ._planner import PlannedProgram, plan_graph
from .dtypes import BFLOAT16, as_dtype, bf16_to_float32, dtype_code, dtype_name
from .lazy import CompiledProgram, Compiler, DeviceAdapter, LazyNode, topological_sort
from .llama import rope_cos_sin


class HIPArray:
    """A device buffer with a shape and dtype (the ``hip`` native type).

    Owns its allocation unless ``base`` is set (a view keeps its base alive).
    Memory returns to the library's caching pool when the array is dropped.
    """

    __slots__ = ("ptr", "shape", "dtype", "base", "_lib", "__weakref__")

    def __init__(self, ptr: Optional[int], shape: Sequence[int], dtype: object,
                 *, base: Optional["HIPArray"] = None, lib=None) -> None:
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.base = base
        self._lib = lib

    @property
    def size(self) -> int:
        result = 1
        for s in self.shape:
            result *= s
        return result

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    def reshape(self, *shape) -> "HIPArray":
        dims = tuple(shape[0]) if len(shape) == 1 and not isinstance(shape[0], int) else tuple(shape)
        if -1 in dims:
            known = int(np.prod([d for d in dims if d != -1]))
            dims = tuple(self.size // known if d == -1 else d for d in dims)
        if int(np.prod(dims)) != self.size:
            raise ValueError("cannot reshape a HIPArray to a different size")
        return HIPArray(self.ptr, dims, self.dtype, base=self.base or self, lib=self._lib)

    def numpy(self) -> np.ndarray:
        return get_device().to_numpy(self)

    def __del__(self) -> None:
        if self.base is None and self.ptr and self._lib is not None:
            try:
                self._lib.raw.chip_free(ctypes.c_void_p(self.ptr))
            except Exception:  # interpreter shutdown
                pass

    def __repr__(self) -> str:
        return f"HIPArray(shape={self.shape}, dtype={dtype_name(self.dtype)})"


_DEVICE: Optional["HIPDeviceAdapter"] = None


def get_device() -> "HIPDeviceAdapter":
    if _DEVICE is None:
        raise RuntimeError("the hip device has not been initialised")
    return _DEVICE


class HIPDeviceAdapter(DeviceAdapter):
    name = "hip"
    inference_dtype = np.dtype(np.float16)

    def __init__(self, lib: "_hiplib.Library", device_index: int = 0) -> None:
        self.lib = lib
        self.index = device_index
        info = _hiplib.ChipInfo()
        lib.call("chip_device_info", ctypes.byref(info))
        self.info = {
            "name": info.name.decode(), "arch": info.arch.decode(),
            "compute_units": info.compute_units, "total_memory": info.total_memory,
            "memory_clock_khz": info.memory_clock_khz, "memory_bus_width": info.memory_bus_width,
        }

    # -- allocation and transfers ---------------------------------------------
    def empty(self, shape: Sequence[int], dtype: object) -> HIPArray:
        dtype = np.dtype(dtype)
        dtype_code(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        if nbytes == 0:
            return HIPArray(None, shape, dtype, lib=self.lib)
        ptr = ctypes.c_void_p()
        self.lib.call("chip_malloc", ctypes.c_size_t(nbytes), ctypes.byref(ptr))
        return HIPArray(ptr.value, shape, dtype, lib=self.lib)

    def array(self, value: object) -> HIPArray:
        if isinstance(value, HIPArray):
            return value
        host = np.asarray(value)
        if host.dtype == np.float64:
            raise TypeError("the hip backend does not support float64; create this tensor as float32")
        if host.dtype == np.bool_:
            host = host.astype(np.int32)
        dtype_code(host.dtype)
        shape = host.shape
        host = np.ascontiguousarray(host)  # (0-d arrays come back 1-d)
        result = self.empty(shape, host.dtype)
        if result.ptr:
            self.lib.call("chip_memcpy_h2d", ctypes.c_void_p(result.ptr),
                          host.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(host.nbytes), 1)
        return result

    def upload(self, dst: HIPArray, value: object) -> None:
        """Queue a copy of a host array into an existing device array of the
        same size (staged through pinned memory; the host array may be reused
        at once).  No allocation, so a loop's bound inputs keep their
        addresses."""
        host = np.ascontiguousarray(as_dtype(np.asarray(value), dst.dtype))
        if host.nbytes != dst.nbytes:
            raise ValueError(f"upload of {host.nbytes} bytes into a {dst.nbytes}-byte array")
        if host.nbytes:
            self.lib.call("chip_memcpy_h2d", ctypes.c_void_p(dst.ptr), host.ctypes.data_as(ctypes.c_void_p),
                          ctypes.c_size_t(host.nbytes), 1)

    def view(self, base: HIPArray, offset: int, shape: Sequence[int]) -> HIPArray:
        """Elements ``offset .. offset + prod(shape)`` of ``base`` as an array
        of ``shape`` (no copy; keeps ``base`` alive)."""
        count = int(np.prod(shape, dtype=np.int64))
        if offset < 0 or offset + count > base.size:
            raise ValueError("view outside its base array")
        return HIPArray(base.ptr + offset * base.dtype.itemsize, shape, base.dtype, base=base, lib=self.lib)

    def zeros(self, shape: Sequence[int], dtype: object) -> HIPArray:
        result = self.empty(shape, dtype)
        if result.ptr:
            self.lib.call("chip_memset", ctypes.c_void_p(result.ptr), 0, ctypes.c_size_t(result.nbytes))
        return result

    def copy(self, value: HIPArray) -> HIPArray:
        result = self.empty(value.shape, value.dtype)
        if result.ptr:
            self.lib.call("chip_memcpy_d2d", ctypes.c_void_p(result.ptr), ctypes.c_void_p(value.ptr),
                          ctypes.c_size_t(value.nbytes))
        return result

    def evaluate(self, values: Sequence[object]) -> None:
        self.synchronize()

    def synchronize(self) -> None:
        self.lib.call("chip_synchronize")

    def to_numpy(self, value: object) -> np.ndarray:
        if not isinstance(value, HIPArray):
            return np.asarray(value)
        host = np.empty(value.shape, dtype=value.dtype)
        if value.nbytes:
            self.lib.call("chip_memcpy_d2h", host.ctypes.data_as(ctypes.c_void_p),
                          ctypes.c_void_p(value.ptr), ctypes.c_size_t(value.nbytes))
        self.lib.call("chip_synchronize")
        return host

    def _argmax_rows(self, value: HIPArray, rows: int, cols: int) -> np.ndarray:
        if cols == 0:
            raise ValueError("attempt to get argmax of an empty sequence")
        out = np.empty(rows, dtype=np.int64)
        self.lib.call("chip_argmax", ctypes.c_void_p(value.ptr), dtype_code(value.dtype),
                      ctypes.c_int64(rows), ctypes.c_int64(cols),
                      out.ctypes.data_as(_hiplib.c_int64_p))
        return out

    def argmax(self, value: object) -> int:
        if not isinstance(value, HIPArray):
            return int(np.asarray(value).argmax())
        return int(self._argmax_rows(value, 1, value.size)[0])

    def argmax_last_axis(self, value: object) -> np.ndarray:
        if not isinstance(value, HIPArray):
            return np.asarray(value).argmax(axis=-1)
        if value.ndim == 0:
            return np.asarray(0)
        cols = value.shape[-1]
        rows = value.size // cols if cols else 0
        if rows == 0:
            return np.zeros(value.shape[:-1], dtype=np.int64)
        return self._argmax_rows(value, rows, cols).reshape(value.shape[:-1])

    def dtype(self, value: object) -> np.dtype:
        return np.dtype(value.dtype)

    # -- weights -------------------------------------------------------------------
    def load_safetensors(self, path: Path, *, dtype: Optional[np.dtype] = None) -> Mapping[str, HIPArray]:
        """Read a .safetensors file (JSON header + raw little-endian tensors),
        convert on the host when ``dtype`` asks for it, upload each tensor.

        Format: 8-byte header length, JSON ``{name: {dtype, shape,
        data_offsets}}``, then the data block (the layout the reference's
        Core ML plugin parses, coreml_backend.py:21-54).  F32, F16 and BF16
        tensors are supported; ``dtype`` may be float32, float16 or bfloat16.
        """
        return {name: self.array(host) for name, host in read_safetensors(path, dtype).items()}

    def reset_peak_memory(self) -> None:
        self.lib.call("chip_reset_peak_memory")

    def peak_memory_bytes(self) -> Optional[int]:
        out = ctypes.c_size_t(0)
        self.lib.call("chip_peak_memory", ctypes.byref(out))
        return int(out.value)

    # -- decode helpers ----------------------------------------------------------------
    def greedy_advance(self, logits: HIPArray, tokens: HIPArray, *, history: Optional[HIPArray] = None,
                       step: int = 0, position: Optional[HIPArray] = None,
                       attention_mask: Optional[HIPArray] = None,
                       write_mask: Optional[HIPArray] = None, cache_length: int = 0) -> None:
        """Queue device-side greedy sampling feeding the next decode step
        (chip_greedy_advance): tokens[r] = argmax(logits[r]); position += 1;
        masks moved to the new position.  Nothing is copied to the host."""
        rows = tokens.size
        cols = logits.size // rows
        mask_dtype = attention_mask.dtype if attention_mask is not None else (
            write_mask.dtype if write_mask is not None else logits.dtype)
        self.lib.call(
            "chip_greedy_advance", ctypes.c_void_p(logits.ptr), dtype_code(logits.dtype),
            ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_void_p(tokens.ptr),
            ctypes.c_void_p(history.ptr if history is not None else None), ctypes.c_int64(step),
            ctypes.c_void_p(position.ptr if position is not None else None),
            ctypes.c_void_p(attention_mask.ptr if attention_mask is not None else None),
            ctypes.c_int64(attention_mask.shape[-1] if attention_mask is not None else 0),
            ctypes.c_void_p(write_mask.ptr if write_mask is not None else None),
            ctypes.c_int64(write_mask.shape[-2] if write_mask is not None else 0),
            dtype_code(mask_dtype), ctypes.c_int64(cache_length))


_SAFETENSORS_TYPES = {"F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "BF16": BFLOAT16,
                      "I32": np.dtype("<i4"), "I64": np.dtype("<i8")}


def read_safetensors(path: Path, dtype: Optional[np.dtype] = None) -> Dict[str, np.ndarray]:
    """Host arrays of a .safetensors file (memory-mapped, converted on request)."""
    requested = np.dtype(dtype) if dtype is not None else None
    if requested is not None and requested not in (np.dtype(np.float32), np.dtype(np.float16), BFLOAT16):
        raise TypeError(f"unsupported hip weight dtype: {requested}")
    with open(path, "rb") as handle:
        header_length = struct.unpack("<Q", handle.read(8))[0]
        if header_length > 100 * 1024 * 1024:
            raise ValueError("safetensors header is implausibly large")
        header = json.loads(handle.read(header_length))
        data = mmap.mmap(handle.fileno(), 0, access=mmap.ACCESS_READ)
    base = 8 + header_length
    result: Dict[str, np.ndarray] = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        kind = meta["dtype"]
        if kind not in _SAFETENSORS_TYPES:
            raise TypeError(f"unsupported safetensors dtype {kind} for {name}")
        begin, end = meta["data_offsets"]
        stored = _SAFETENSORS_TYPES[kind]
        shape = tuple(meta["shape"])
        count = int(np.prod(shape, dtype=np.int64))
        if end - begin != count * stored.itemsize:
            raise ValueError(f"safetensors entry {name} has inconsistent offsets")
        array = np.frombuffer(data, dtype=stored, count=count, offset=base + begin).reshape(shape)
        if requested is not None and array.dtype != requested and kind in ("F32", "F16", "BF16"):
            source = bf16_to_float32(array) if array.dtype == BFLOAT16 else array.astype(np.float32)
            array = as_dtype(source, requested)
        else:
            array = np.array(array)
        result[name] = array
    return result


class HIPProgram(CompiledProgram):
    """A planned graph bound to a ``chip_plan`` (one hipGraph per run)."""

    def __init__(self, compiler: "HIPCompiler", planned: PlannedProgram, owner: "_PlanHandle",
                 inputs: Tuple[LazyNode, ...], leaf_map: Dict[LazyNode, LazyNode]):
        self._compiler = compiler
        self._planned = planned
        # Programs of one structure share the plan (the structural program
        # cache), so what is bound to it is recorded on the shared owner,
        # never per program: another program may have rebound it since.
        self._handle_owner = owner
        self._plan = owner.handle
        self.device = compiler.device
        self.inputs = inputs
        self.source = planned.source
        self._leaf_map = leaf_map          # this graph's leaf -> planned leaf

    @property
    def kernel_count(self) -> int:
        return len(self._planned.steps)

    def _bind(self, slots: List[int], pointers: List[int]) -> None:
        bound = self._handle_owner.bound
        changed = [(s, p) for s, p in zip(slots, pointers) if bound.get(s) != p]
        if not changed or self._plan is None:
            return
        n = len(changed)
        slot_array = (ctypes.c_uint32 * n)(*[s for s, _ in changed])
        ptr_array = (ctypes.c_void_p * n)(*[p for _, p in changed])
        self._compiler.lib.call("chip_plan_bind_many", self._plan, ctypes.c_uint32(n), slot_array, ptr_array)
        for s, p in changed:
            bound[s] = p

    def run(
        self,
        bindings: Optional[Mapping[LazyNode, object]] = None,
        *,
        synchronize: bool = False,
        out: Optional[Sequence[Optional[HIPArray]]] = None,
    ) -> Tuple[object, ...]:
        """Queue one execution.  ``bindings`` replaces inputs (device arrays,
        or host arrays which are uploaded); ``out`` may supply preallocated
        output arrays (entries for leaf or donated outputs are ignored)."""
        replacements = bindings or {}
        planned = self._planned
        # Resident loops run the same device arrays step after step: then
        # nothing needs checking or binding again, provided this program made
        # the plan's last run (the owner records which one did).
        run_arrays: Optional[Tuple[object, ...]] = None
        if all(isinstance(replacements.get(node), HIPArray) for node in self.inputs):
            run_arrays = tuple(replacements[node] for node in self.inputs) + tuple(out or ())
            last = self._handle_owner.repeat
            if (last is not None and last[0] is self and len(last[1]) == len(run_arrays)
                    and all(a is b for a, b in zip(last[1], run_arrays))):
                if self._plan is not None:
                    self._compiler.lib.call("chip_plan_run", self._plan)
                if synchronize:
                    self.device.synchronize()
                return last[2]
        natives: Dict[LazyNode, HIPArray] = {}
        slots: List[int] = []
        pointers: List[int] = []
        for node in self.inputs:
            value = replacements[node] if node in replacements else self._compiler._load_input(node)
            if not isinstance(value, HIPArray):
                value = self.device.array(as_dtype(value, node.dtype))
            if value.shape != node.shape or value.dtype != node.dtype:
                raise ValueError(
                    f"binding for input {node.shape} {dtype_name(node.dtype)} has shape "
                    f"{value.shape} and dtype {dtype_name(value.dtype)}"
                )
            planned_leaf = self._leaf_map[node]
            natives[planned_leaf] = value
            slot = planned.input_slots.get(planned_leaf)
            if slot is not None:
                if value.ptr is None:
                    raise ValueError("an empty array cannot be bound to a planned input")
                slots.append(slot)
                pointers.append(value.ptr)

        results: List[object] = []
        fresh: Dict[int, HIPArray] = {}
        fresh_made = False
        for index, (kind, payload) in enumerate(planned.output_specs):
            node = planned.output_nodes[index]
            if kind == "empty":
                results.append(HIPArray(None, node.shape, node.dtype, lib=self._compiler.lib))
            elif kind == "input":
                results.append(natives[payload])
            elif kind == "const":
                results.append(payload)
            else:
                storage = payload
                array = fresh.get(id(storage))
                if array is None:
                    given = out[index] if out is not None and index < len(out) else None
                    if given is not None:
                        if given.nbytes != storage.nbytes:
                            raise ValueError("preallocated output has the wrong size")
                        array = given if given.shape == node.shape else given.reshape(node.shape)
                    else:
                        array = self.device.empty(node.shape, node.dtype)
                        fresh_made = True
                    fresh[id(storage)] = array
                    slots.append(storage.slot)
                    pointers.append(array.ptr)
                results.append(array)
        if self._plan is not None:
            self._bind(slots, pointers)
            self._compiler.lib.call("chip_plan_run", self._plan)
        if synchronize:
            self.device.synchronize()
        # remember the run for repeats when no output array was made here
        # (a fresh array per run is what a caller without ``out`` gets); the
        # arrays stay referenced, so their ids cannot be reused meanwhile
        self._handle_owner.repeat = (
            (self, run_arrays, tuple(results)) if run_arrays is not None and not fresh_made else None)
        return tuple(results)


class _PlanHandle:
    """Owns a chip_plan and the constants its kernels read."""

    def __init__(self, lib, planned: PlannedProgram) -> None:
        self.lib = lib
        self.handle = None
        self.constants = list(planned.constants)
        self.bound: Dict[int, int] = {}  # slot -> pointer bound last, by any program of this plan
        # (program, its input and output arrays, results) of the last run
        # that a repeat with the same arrays may reuse as is
        self.repeat: Optional[Tuple[object, Tuple[object, ...], Tuple[object, ...]]] = None
        if not planned.steps:
            return
        tape = np.ascontiguousarray(planned.tape, dtype=np.int64)
        handle = ctypes.c_void_p()
        lib.call("chip_plan_create", tape.ctypes.data_as(_hiplib.c_int64_p),
                 ctypes.c_size_t(tape.size), ctypes.byref(handle))
        self.handle = handle
        slots, pointers = [], []
        for storage in planned.storages:
            if storage.kind == "const" and storage.slot > 0:
                slots.append(storage.slot)
                pointers.append(storage.native.ptr)
        if slots:
            n = len(slots)
            lib.call("chip_plan_bind_many", handle, ctypes.c_uint32(n),
                     (ctypes.c_uint32 * n)(*slots), (ctypes.c_void_p * n)(*pointers))

    def __del__(self) -> None:
        if self.handle is not None:
            try:
                self.lib.raw.chip_plan_destroy(self.handle)
            except Exception:
                pass


class HIPCompiler(Compiler):
    """Compile lazy graphs into gfx950 kernel plans."""

    def __init__(self) -> None:
        global _DEVICE
        self.lib = _hiplib.load()
        index = int(os.environ.get("CHOMIK_HIP_DEVICE", "0"))
        self.lib.call("chip_init", index)
        if _DEVICE is None:
            _DEVICE = HIPDeviceAdapter(self.lib, index)
        self.device = _DEVICE
        self._program_cache: Dict[object, Tuple[PlannedProgram, _PlanHandle]] = {}
        self._rope_tables: Dict[Tuple, HIPArray] = {}

    @property
    def cache_size(self) -> int:
        return len(self._program_cache)

    def close(self) -> None:
        self.device.synchronize()
        self._program_cache.clear()

    def _load_input(self, node: LazyNode) -> HIPArray:
        native = node.native_values.get("hip")
        if native is not None:
            return native
        native = self.device.array(as_dtype(node.numpy_value(), node.dtype))
        if node.cache_native:
            node.native_values["hip"] = native
        return native

    def _rope_table(self, head: int, theta: float, dtype: np.dtype, length: int) -> HIPArray:
        """(length, head) table: row p holds cos then sin of p * theta^(-2i/head),
        rounded to the model dtype exactly as the portable rotation matrix."""
        key = (head, theta, np.dtype(dtype).str)
        table = self._rope_tables.get(key)
        if table is None or table.shape[0] < length:
            cosine, sine = rope_cos_sin(np.arange(length, dtype=np.float32), head, theta)
            host = as_dtype(np.concatenate([cosine, sine], axis=1), dtype)
            table = self.device.array(host)
            self._rope_tables[key] = table
        return table

    def compile(
        self,
        outputs: Sequence[LazyNode],
        dynamic_inputs: Sequence[LazyNode] = (),
        *,
        donate: Sequence[LazyNode] = (),
    ) -> HIPProgram:
        """Compile ``outputs``.  ``donate`` (an extension) lists dynamic KV-cache
        inputs whose buffers the program may update in place: the returned
        cache then *is* the bound input array.  Without it caches are
        functional, as in the reference."""
        if not outputs:
            raise ValueError("at least one output is required")
        if any(node.op is not None for node in dynamic_inputs):
            raise ValueError("dynamic inputs must be graph leaves")
        requested = set(dynamic_inputs)
        if not set(donate).issubset(requested):
            raise ValueError("donated inputs must be dynamic inputs")
        portable = {n for n in topological_sort(outputs) if n.op is None}
        lowered = {n for n in topological_sort(outputs, use_lowerings=True) if n.op is None}
        if not requested.issubset(portable | lowered):
            raise ValueError("dynamic input is not a leaf of the compiled graph")

        specialized = bool(dynamic_inputs)
        if not specialized:
            from ._planner import choose_lowerings
            plan = choose_lowerings(outputs, set())
            signature = plan.signature()
            cached = self._program_cache.get(signature)
            if cached is not None:
                planned, handle = cached
                leaves = tuple(n for n in plan.nodes() if n.op is None)
                leaf_map = dict(zip(leaves, planned.leaves))
                return HIPProgram(self, planned, handle, leaves, leaf_map)

        planned = plan_graph(self, outputs, dynamic_inputs, donate)
        handle = _PlanHandle(self.lib, planned)
        if specialized:
            inputs = tuple(n for n in planned.leaves if n in requested)
        else:
            inputs = planned.leaves
            self._program_cache[planned.signature] = (planned, handle)
        leaf_map = {n: n for n in planned.leaves}
        return HIPProgram(self, planned, handle, inputs, leaf_map)


def register_into(lazy_module, *, replace: bool = False) -> None:
    """Register the ``hip`` plugin into another copy of the plugin API.

    ``lazy_module`` is a module with the reference's registry and plugin
    ABCs (``register_compiler``, ``Compiler``, ``CompiledProgram``,
    ``DeviceAdapter``; chomikgrad/lazy.py:107-209, 646-678), such as the
    reference package's own ``chomikgrad.lazy``.  Its ``get_compiler`` checks
    ``isinstance(compiler, Compiler)`` against its own ABC, so the plugin's
    classes are registered there as virtual subclasses.  Graphs built from
    that module's ``LazyNode`` and ``Op`` are planned by operation value
    (``lazy.op_of``); natives are stored under ``native_values["hip"]``, the
    name registered here, so that module's ``LazyNode.numpy_value`` reads
    them back through this plugin's adapter.
    """
    lazy_module.Compiler.register(HIPCompiler)
    lazy_module.CompiledProgram.register(HIPProgram)
    lazy_module.DeviceAdapter.register(HIPDeviceAdapter)
    lazy_module.register_compiler("hip", HIPCompiler, replace=replace)
