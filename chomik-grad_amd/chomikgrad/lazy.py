"""The six-op lazy IR, the compiler-plugin contract and the plugin registry.

This module restates the public surface of the reference's
chomikgrad/lazy.py so that graphs built here and plugins written against it
behave the same way:

* ``Op`` and ``LazyNode``            -- chomikgrad/lazy.py:22-104
* ``DeviceAdapter``                  -- chomikgrad/lazy.py:107-151
* ``CompiledProgram``                -- chomikgrad/lazy.py:154-169
* ``Compiler``                       -- chomikgrad/lazy.py:172-209
* ``topological_sort``               -- chomikgrad/lazy.py:212-233
* ``GraphPlan``                      -- chomikgrad/lazy.py:236-378
* registry (``register_compiler``,
  ``set_default_compiler``,
  ``get_compiler``, ``realize_nodes``) -- chomikgrad/lazy.py:639-684

The NumPy ``cpu`` plugin that the reference registers in the same file is
the correctness oracle of this build and lives outside the product package.
The default compiler here is therefore ``hip``.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from enum import Enum
from pathlib import Path
from typing import (
    Callable,
    Dict,
    Iterable,
    List,
    Mapping,
    Optional,
    Sequence,
    Tuple,
    Union,
)

import numpy as np

Lowering = Tuple[str, Tuple["LazyNode", ...], object]


class Op(Enum):
    """The whole instruction set.  Variants (add, exp, sum, ...) are args."""

    ELEMENTWISE = "elementwise"
    REDUCE = "reduce"
    RESHAPE = "reshape"
    PERMUTE = "permute"
    MATMUL = "matmul"
    GATHER = "gather"


def op_of(node: "LazyNode") -> Optional[Op]:
    """The node's operation as this module's ``Op``, or None for a leaf.

    Nodes built by another copy of the IR (for example the reference
    package's own ``chomikgrad.lazy``, whose ``Op`` has the same member
    names and values but is a different class) are matched by value, so a
    plugin registered into that package's registry plans its graphs too.
    """
    op = node.op
    if op is None or type(op) is Op:
        return op
    return Op(op.value)


class LazyNode:
    """One value of a lazy graph.

    A leaf has ``op is None`` and carries either a host ``value`` or backend
    natives in ``native_values`` (backend name -> native array).  An optional
    ``lowering = (kind, inputs, argument)`` names a fused form a plugin may
    execute instead of the portable expansion below this node.
    """

    __slots__ = (
        "op",
        "inputs",
        "arg",
        "shape",
        "dtype",
        "value",
        "native_values",
        "cache_native",
        "lowering",
    )

    def __init__(
        self,
        op: Optional[Op],
        inputs: Sequence["LazyNode"],
        arg: object,
        shape: Sequence[int],
        dtype: object,
        value: Optional[np.ndarray] = None,
        native_values: Optional[Dict[str, object]] = None,
        cache_native: bool = True,
        lowering: Optional[Lowering] = None,
    ) -> None:
        self.op = op
        self.inputs = tuple(inputs)
        self.arg = arg
        self.shape = tuple(int(size) for size in shape)
        self.dtype = np.dtype(dtype)
        self.value = value
        self.native_values = {} if native_values is None else native_values
        self.cache_native = cache_native
        self.lowering = lowering

    @classmethod
    def leaf(cls, value: np.ndarray, *, cache_native: bool = True) -> "LazyNode":
        return cls(
            None, (), None, value.shape, value.dtype, value,
            cache_native=cache_native,
        )

    @classmethod
    def native_leaf(
        cls, backend: str, value: object, shape: Sequence[int], dtype: object
    ) -> "LazyNode":
        return cls(None, (), None, shape, dtype, native_values={backend: value})

    @property
    def is_leaf(self) -> bool:
        return self.op is None

    def numpy_value(self) -> np.ndarray:
        """Host value of a leaf, reading a native back through its adapter."""
        if self.value is not None:
            return self.value
        if not self.native_values:
            raise RuntimeError("leaf node has no value")
        backend, native = next(iter(self.native_values.items()))
        try:
            host = get_compiler(backend).device.to_numpy(native)
        except KeyError:
            host = native
        self.value = np.array(host, copy=True)
        return self.value

    def __repr__(self) -> str:
        kind = "leaf" if self.op is None else self.op.value
        return f"LazyNode({kind}, shape={self.shape}, dtype={self.dtype})"


class DeviceAdapter(ABC):
    """The runtime boundary a compiled backend exposes to drivers."""

    name: str

    @abstractmethod
    def array(self, value: object) -> object:
        """Upload host data and return a native array."""

    @abstractmethod
    def evaluate(self, values: Sequence[object]) -> None:
        """Make the given natives ready (complete any pending work)."""

    @abstractmethod
    def synchronize(self) -> None:
        """Wait for all work queued on the device."""

    @abstractmethod
    def to_numpy(self, value: object) -> np.ndarray:
        """Copy a native back to the host (synchronises)."""

    @abstractmethod
    def argmax(self, value: object) -> int:
        """Index of the first maximum of the flattened native (synchronises)."""

    def argmax_last_axis(self, value: object) -> np.ndarray:
        return np.asarray(self.to_numpy(value)).argmax(axis=-1)

    @abstractmethod
    def dtype(self, value: object) -> np.dtype:
        """Element type of a native."""

    def load_safetensors(
        self, path: Path, *, dtype: Optional[np.dtype] = None
    ) -> Mapping[str, object]:
        raise NotImplementedError(
            f"the {self.name!r} device does not support safetensors loading"
        )

    def reset_peak_memory(self) -> None:
        pass

    def peak_memory_bytes(self) -> Optional[int]:
        return None


class CompiledProgram(ABC):
    """An executable graph.  ``run`` may return before the device finishes."""

    source: str
    device: DeviceAdapter

    @abstractmethod
    def run(
        self,
        bindings: Optional[Mapping[LazyNode, object]] = None,
        *,
        synchronize: bool = False,
    ) -> Tuple[object, ...]:
        """Execute; unbound inputs take their leaf's cached native/value."""

    def __call__(self) -> Tuple[np.ndarray, ...]:
        outputs = self.run(synchronize=True)
        return tuple(self.device.to_numpy(output) for output in outputs)


class Compiler(ABC):
    """A plugin translating lazy nodes into a ``CompiledProgram``."""

    device: DeviceAdapter

    @abstractmethod
    def compile(
        self,
        outputs: Sequence[LazyNode],
        dynamic_inputs: Sequence[LazyNode] = (),
    ) -> CompiledProgram:
        """Compile ``outputs``.

        Without ``dynamic_inputs`` every leaf is a program input.  With them,
        only those leaves are inputs and every other leaf is captured once at
        compile time (weights).
        """

    def update_parameters(
        self,
        parameters: Sequence[LazyNode],
        gradients: Sequence[LazyNode],
        learning_rate: float,
        *,
        inplace: bool = False,
    ) -> Optional[Tuple[Tuple[LazyNode, ...], Tuple[LazyNode, ...]]]:
        if inplace:
            raise RuntimeError(
                "this compiler does not support in-place parameter updates"
            )
        return None

    def update_native_parameters(
        self,
        parameters: Sequence[LazyNode],
        gradients: Sequence[object],
        learning_rate: float,
        *,
        inplace: bool = False,
    ) -> Tuple[Tuple[LazyNode, ...], Tuple[LazyNode, ...]]:
        raise RuntimeError("this compiler does not support compiled training steps")


def _ordered(
    outputs: Iterable[LazyNode], parents: Callable[[LazyNode], Sequence[LazyNode]]
) -> Tuple[LazyNode, ...]:
    """Post-order DFS (parents before children), iterative so deep graphs
    such as a 22-layer decode step never hit Python's recursion limit."""
    order: List[LazyNode] = []
    seen = set()
    for root in outputs:
        if root in seen:
            continue
        seen.add(root)
        stack = [(root, iter(parents(root)))]
        while stack:
            node, pending = stack[-1]
            advanced = False
            for parent in pending:
                if parent not in seen:
                    seen.add(parent)
                    stack.append((parent, iter(parents(parent))))
                    advanced = True
                    break
            if not advanced:
                stack.pop()
                order.append(node)
    return tuple(order)


def topological_sort(
    outputs: Iterable[LazyNode], *, use_lowerings: bool = False
) -> Tuple[LazyNode, ...]:
    if use_lowerings:
        return _ordered(
            outputs,
            lambda node: node.lowering[1] if node.lowering is not None else node.inputs,
        )
    return _ordered(outputs, lambda node: node.inputs)


class GraphPlan:
    """Backend-local view of a graph: which lowerings are taken, and fusions.

    Choosing a lowering never mutates a ``LazyNode``: intrinsic tags are
    honoured only when listed in ``supported_lowerings`` and plan-local
    rewrites live in ``_overrides``.
    """

    def __init__(
        self, outputs: Sequence[LazyNode], supported_lowerings: Iterable[str]
    ) -> None:
        if not outputs:
            raise ValueError("at least one output is required")
        self.outputs = tuple(outputs)
        self.supported_lowerings = frozenset(supported_lowerings)
        self._overrides: Dict[LazyNode, Lowering] = {}

    def lowering(self, node: LazyNode) -> Optional[Lowering]:
        override = self._overrides.get(node)
        if override is not None:
            return override
        tag = node.lowering
        if tag is not None and tag[0] in self.supported_lowerings:
            return tag
        return None

    def override(self, node: LazyNode, lowering: Lowering) -> None:
        self._overrides[node] = lowering

    def inputs(self, node: LazyNode) -> Tuple[LazyNode, ...]:
        chosen = self.lowering(node)
        return tuple(chosen[1]) if chosen is not None else node.inputs

    def nodes(self) -> Tuple[LazyNode, ...]:
        return _ordered(self.outputs, self.inputs)

    def signature(self, nodes: Optional[Sequence[LazyNode]] = None) -> object:
        """Structural key: equal for graphs that differ only in leaf values.

        Leaf identity is positional, so ``a + a`` and ``a + b`` differ.
        """
        chosen = tuple(nodes) if nodes is not None else self.nodes()
        index = {node: position for position, node in enumerate(chosen)}
        entries = []
        for node in chosen:
            lowering = self.lowering(node)
            if node.op is None:
                entries.append((None, node.shape, node.dtype.str))
            elif lowering is not None:
                kind, parents, argument = lowering
                entries.append(
                    ("lowering", kind, repr(argument), node.shape, node.dtype.str,
                     tuple(index[parent] for parent in parents))
                )
            else:
                entries.append(
                    (node.op.value, repr(node.arg), node.shape, node.dtype.str,
                     tuple(index[parent] for parent in node.inputs))
                )
        return tuple(entries), tuple(index[node] for node in self.outputs)

    def fuse_elementwise(self) -> None:
        """Fold single-consumer, same-shape ELEMENTWISE chains into one
        ``("elementwise_fusion", inputs, expression)`` override per root.

        The expression is a nested tuple ``(kind, dtype_str, *children)`` with
        ``("input", i)`` leaves.  Each step keeps its own dtype, so a fused
        float16 chain still rounds after every operation.
        """
        nodes = self.nodes()
        consumers: Dict[LazyNode, int] = {}
        for node in nodes:
            for parent in self.inputs(node):
                consumers[parent] = consumers.get(parent, 0) + 1
        outputs = set(self.outputs)

        def eligible(node: LazyNode) -> bool:
            return (
                op_of(node) is Op.ELEMENTWISE
                and self.lowering(node) is None
                and _float_dtype(node.dtype)
            )

        absorbed = set()
        for child in nodes:
            if not eligible(child):
                continue
            for parent in child.inputs:
                if (
                    eligible(parent)
                    and parent.shape == child.shape
                    and consumers.get(parent) == 1
                    and parent not in outputs
                ):
                    absorbed.add(parent)

        for root in nodes:
            if not eligible(root) or root in absorbed:
                continue
            operands: List[LazyNode] = []
            operand_index: Dict[LazyNode, int] = {}
            fused = 0

            def expand(node: LazyNode) -> tuple:
                nonlocal fused
                if node is root or node in absorbed:
                    fused += 1
                    return (str(node.arg), node.dtype.str) + tuple(
                        expand(parent) for parent in node.inputs
                    )
                if node not in operand_index:
                    operand_index[node] = len(operands)
                    operands.append(node)
                return ("input", operand_index[node])

            expression = expand(root)
            if fused > 1:
                self._overrides[root] = (
                    "elementwise_fusion", tuple(operands), expression,
                )


def _float_dtype(dtype: np.dtype) -> bool:
    from .dtypes import is_float

    return is_float(dtype) and dtype != np.dtype(np.float64)


CompilerFactory = Callable[[], Compiler]
CompilerRegistration = Union[Compiler, CompilerFactory]
_COMPILERS: Dict[str, CompilerRegistration] = {}
_COMPILER_INSTANCES: Dict[str, Compiler] = {}
_DEFAULT_COMPILER = "hip"


def register_compiler(
    name: str, compiler: CompilerRegistration, *, replace: bool = False
) -> None:
    """Register a compiler instance or a zero-argument factory (a class)."""
    if not name:
        raise ValueError("compiler name cannot be empty")
    if name in _COMPILERS and not replace:
        raise ValueError(f"compiler already registered: {name}")
    if not isinstance(compiler, Compiler) and not callable(compiler):
        raise TypeError("compiler must be a Compiler instance or a factory")
    _COMPILERS[name] = compiler
    _COMPILER_INSTANCES.pop(name, None)


def set_default_compiler(name: str) -> None:
    global _DEFAULT_COMPILER
    if name not in _COMPILERS:
        raise KeyError(f"unknown compiler: {name}")
    _DEFAULT_COMPILER = name


def default_compiler_name() -> str:
    return _DEFAULT_COMPILER


def get_compiler(name: Optional[str] = None) -> Compiler:
    """Return the named compiler, instantiating a factory on first use."""
    selected = name or _DEFAULT_COMPILER
    instance = _COMPILER_INSTANCES.get(selected)
    if instance is not None:
        return instance
    if selected not in _COMPILERS:
        raise KeyError(f"unknown compiler: {selected}")
    registration = _COMPILERS[selected]
    compiler = registration if isinstance(registration, Compiler) else registration()
    if not isinstance(compiler, Compiler):
        raise TypeError(f"compiler factory {selected!r} returned an invalid object")
    _COMPILER_INSTANCES[selected] = compiler
    return compiler


def realize_nodes(
    outputs: Sequence[LazyNode], compiler: Optional[str] = None
) -> Tuple[np.ndarray, ...]:
    return get_compiler(compiler).compile(outputs)()
