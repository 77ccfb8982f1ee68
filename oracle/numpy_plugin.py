"""The NumPy ``cpu`` plugin, restated as the oracle -- TEST INFRASTRUCTURE ONLY.

Follows the reference's ``NumpyCompiler`` (chomikgrad/lazy.py:551-636):
every node is evaluated with the NumPy routine the reference's generated code
calls, on the portable graph (lowering tags are ignored):

=============  =====================================================
ELEMENTWISE    np.add / np.subtract / np.multiply / np.divide,
               np.equal(...).astype(left dtype), np.negative, np.exp,
               np.log, np.sqrt, np.maximum(x, 0),
               np.greater(x, 0).astype(x dtype)        (lazy.py:554-568)
REDUCE         np.sum / np.max(axis=axes, keepdims=k)   (lazy.py:618-622)
RESHAPE        np.reshape                               (lazy.py:624-625)
PERMUTE        np.transpose(axes=...)                   (lazy.py:627-628)
MATMUL         np.matmul                                (lazy.py:630-631)
GATHER         np.take(table, ids, axis=0)              (lazy.py:633-634)
=============  =====================================================

float16 therefore rounds after every elementwise op, while np.matmul and
np.sum accumulate in float32 and round once (NumPy's half loops).

bfloat16 has no NumPy type and the reference would need ``ml_dtypes``
(pyproject.toml:29-33), which is absent.  bf16 values (the two-byte
``BFLOAT16`` marker dtype) are emulated with the float16 rules: each op is
computed in float32 from the bf16 inputs and rounded once to bf16, nearest
even (``_to_bf16`` below, checked against torch's CPU bfloat16 in tests).
No reference test covers bf16, so bf16 parity is pinned only by that
conversion check and by the properties the tests assert.

Inputs are all leaves in topological order and any leaf may be rebound, as
in the reference (lazy.py:509-525).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np

from chomikgrad.dtypes import BFLOAT16
from chomikgrad.lazy import (
    CompiledProgram,
    Compiler,
    DeviceAdapter,
    LazyNode,
    Op,
    register_compiler,
    topological_sort,
)


def _to_bf16(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 marker array, round to nearest, ties to even."""
    f32 = np.ascontiguousarray(values, dtype=np.float32)
    bits = f32.view(np.uint32).astype(np.uint64)
    halfway = np.uint64(0x7FFF) + ((bits >> np.uint64(16)) & np.uint64(1))
    upper = ((bits + halfway) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f32)
    if nan.any():
        upper = np.where(nan, np.uint16(0x7FC0), upper)
    return upper.view(BFLOAT16).reshape(f32.shape)


def _from_bf16(values: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(values).view(np.uint16).astype(np.uint32)
    return (raw << np.uint32(16)).view(np.float32).reshape(values.shape)


def _is_bf16(array: np.ndarray) -> bool:
    return array.dtype == BFLOAT16


_BINARY: Dict[str, Tuple[str, Callable]] = {
    "add": ("np.add({0}, {1})", np.add),
    "sub": ("np.subtract({0}, {1})", np.subtract),
    "mul": ("np.multiply({0}, {1})", np.multiply),
    "div": ("np.divide({0}, {1})", np.divide),
    "equal": ("np.equal({0}, {1}).astype({0}.dtype)",
              lambda a, b: np.equal(a, b).astype(a.dtype, copy=False)),
}
_UNARY: Dict[str, Tuple[str, Callable]] = {
    "neg": ("np.negative({0})", np.negative),
    "exp": ("np.exp({0})", np.exp),
    "log": ("np.log({0})", np.log),
    "sqrt": ("np.sqrt({0})", np.sqrt),
    "relu": ("np.maximum({0}, 0)", lambda a: np.maximum(a, 0)),
    "step": ("np.greater({0}, 0).astype({0}.dtype)",
             lambda a: np.greater(a, 0).astype(a.dtype, copy=False)),
}


def _render(node: LazyNode, names: Sequence[str]) -> str:
    if node.op is Op.ELEMENTWISE:
        table = _BINARY if node.arg in _BINARY else _UNARY
        if node.arg not in table:
            raise ValueError(f"unsupported elementwise operation: {node.arg}")
        return table[node.arg][0].format(*names)
    if node.op is Op.REDUCE:
        kind, axes, keepdims = node.arg
        if kind not in ("sum", "max"):
            raise ValueError(f"unsupported reduction: {kind}")
        return f"np.{kind}({names[0]}, axis={axes!r}, keepdims={keepdims!r})"
    if node.op is Op.RESHAPE:
        return f"np.reshape({names[0]}, {node.arg!r})"
    if node.op is Op.PERMUTE:
        return f"np.transpose({names[0]}, axes={node.arg!r})"
    if node.op is Op.MATMUL:
        return f"np.matmul({names[0]}, {names[1]})"
    if node.op is Op.GATHER:
        return f"np.take({names[0]}, {names[1]}, axis=0)"
    raise ValueError(f"unsupported operation: {node.op}")


def evaluate_node(node: LazyNode, args: Sequence[np.ndarray]) -> np.ndarray:
    """One IR node on NumPy arrays (bf16 emulated as described above)."""
    op = node.op
    if op is Op.RESHAPE:
        return np.reshape(args[0], node.arg)
    if op is Op.PERMUTE:
        return np.transpose(args[0], axes=node.arg)
    if op is Op.GATHER:
        return np.take(args[0], args[1], axis=0)

    emulate = any(_is_bf16(a) for a in args)
    values = [_from_bf16(a) if _is_bf16(a) else a for a in args]
    if op is Op.ELEMENTWISE:
        kind = str(node.arg)
        if kind in _BINARY:
            result = _BINARY[kind][1](values[0], values[1])
        elif kind in _UNARY:
            result = _UNARY[kind][1](values[0])
        else:
            raise ValueError(f"unsupported elementwise operation: {kind}")
    elif op is Op.REDUCE:
        kind, axes, keepdims = node.arg
        if kind == "sum":
            result = np.sum(values[0], axis=axes, keepdims=keepdims)
        elif kind == "max":
            result = np.max(values[0], axis=axes, keepdims=keepdims)
        else:
            raise ValueError(f"unsupported reduction: {kind}")
    elif op is Op.MATMUL:
        result = np.matmul(values[0], values[1])
    else:
        raise ValueError(f"unsupported operation: {op}")
    result = np.asarray(result)
    if emulate and node.dtype == BFLOAT16:
        return _to_bf16(result)
    return result


@dataclass
class NumpyProgram(CompiledProgram):
    source: str
    inputs: Tuple[LazyNode, ...]
    _nodes: Tuple[LazyNode, ...]
    _outputs: Tuple[LazyNode, ...]
    device: DeviceAdapter

    def run(
        self,
        bindings: Optional[Mapping[LazyNode, object]] = None,
        *,
        synchronize: bool = False,
    ) -> Tuple[object, ...]:
        replacements = bindings or {}
        last_use: Dict[LazyNode, int] = {}
        for position, node in enumerate(self._nodes):
            for parent in node.inputs:
                last_use[parent] = position
        keep = set(self._outputs)
        values: Dict[LazyNode, np.ndarray] = {}
        for position, node in enumerate(self._nodes):
            if node.op is None:
                values[node] = (
                    np.asarray(replacements[node]) if node in replacements
                    else node.numpy_value()
                )
            else:
                values[node] = evaluate_node(node, [values[p] for p in node.inputs])
            for parent in set(node.inputs):
                if last_use.get(parent) == position and parent not in keep:
                    del values[parent]
        outputs = tuple(np.asarray(values[node]) for node in self._outputs)
        if synchronize:
            self.device.evaluate(outputs)
        return outputs


class NumpyDeviceAdapter(DeviceAdapter):
    name = "cpu"

    def array(self, value: object) -> np.ndarray:
        return np.asarray(value)

    def evaluate(self, values: Sequence[object]) -> None:
        for value in values:
            np.asarray(value)

    def synchronize(self) -> None:
        pass

    def to_numpy(self, value: object) -> np.ndarray:
        return np.asarray(value)

    def argmax(self, value: object) -> int:
        array = np.asarray(value)
        if _is_bf16(array):
            array = _from_bf16(array)
        return int(array.argmax())

    def argmax_last_axis(self, value: object) -> np.ndarray:
        array = np.asarray(value)
        if _is_bf16(array):
            array = _from_bf16(array)
        return array.argmax(axis=-1)

    def dtype(self, value: object) -> np.dtype:
        return np.asarray(value).dtype


class NumpyCompiler(Compiler):
    """Evaluates the portable graph node by node on the host."""

    def __init__(self) -> None:
        self.device = NumpyDeviceAdapter()

    def compile(
        self,
        outputs: Sequence[LazyNode],
        dynamic_inputs: Sequence[LazyNode] = (),
    ) -> NumpyProgram:
        if not outputs:
            raise ValueError("at least one output is required")
        nodes = topological_sort(outputs)
        names = {node: f"v{i}" for i, node in enumerate(nodes)}
        leaves = tuple(node for node in nodes if node.op is None)
        leaf_index = {node: i for i, node in enumerate(leaves)}
        lines: List[str] = ["def run(inputs):"]
        for node in nodes:
            if node.op is None:
                lines.append(f"    {names[node]} = inputs[{leaf_index[node]}]")
            else:
                lines.append(
                    f"    {names[node]} = {_render(node, [names[p] for p in node.inputs])}"
                )
        rendered = ", ".join(names[node] for node in outputs)
        lines.append(f"    return ({rendered}{',' if len(outputs) == 1 else ''})")
        return NumpyProgram("\n".join(lines), leaves, nodes, tuple(outputs), self.device)


def install(*, replace: bool = True) -> None:
    """Register this oracle as the ``cpu`` compiler."""
    register_compiler("cpu", NumpyCompiler, replace=replace)


install()
