"""Lazy ``Tensor`` front-end: the forward graph constructors.

Graph semantics follow the reference's chomikgrad/tensor.py:
* scalars are coerced to leaves of the tensor's own dtype (tensor.py:205-208);
* binary ops broadcast like NumPy and promote with ``np.result_type``
  (tensor.py:210-244), extended here with the ``BFLOAT16`` marker dtype;
* ``mean`` is ``sum`` divided by the element count (tensor.py:586-589);
* ``softmax`` is ``exp(x - max(x)) / sum`` tagged ``("softmax", (x,), axis)``
  (tensor.py:325-352);
* ``gather`` has shape ``indices.shape + table.shape[1:]`` (tensor.py:527-564);
* ``matmul`` broadcasts batch dimensions (tensor.py:498-525);
* ``compile_graph`` / ``realize`` (tensor.py:623-642).

Autograd (``backward``) belongs to the reference's training path, which this
build does not cover; ``backward`` raises ``NotImplementedError``.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Iterator, Optional, Sequence, Tuple, Union

import numpy as np

from .dtypes import BFLOAT16, as_dtype, is_float, is_integer, result_type
from .lazy import CompiledProgram, LazyNode, Op, get_compiler

ArrayLike = Union[float, int, Sequence[float], np.ndarray]
Axis = Optional[Union[int, Sequence[int]]]

_GRAD_ENABLED = True


@contextmanager
def no_grad() -> Iterator[None]:
    global _GRAD_ENABLED
    saved = _GRAD_ENABLED
    _GRAD_ENABLED = False
    try:
        yield
    finally:
        _GRAD_ENABLED = saved


def _axes(axis: Axis, ndim: int) -> Tuple[int, ...]:
    if axis is None:
        return tuple(range(ndim))
    raw = (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis)
    result = tuple(int(a) + ndim if int(a) < 0 else int(a) for a in raw)
    if any(a < 0 or a >= ndim for a in result):
        raise ValueError(f"axis {axis!r} is invalid for a {ndim}D tensor")
    if len(set(result)) != len(result):
        raise ValueError("reduction axes must be unique")
    return result


def _reduced(shape: Tuple[int, ...], axes: Tuple[int, ...], keepdims: bool) -> Tuple[int, ...]:
    if keepdims:
        return tuple(1 if i in axes else n for i, n in enumerate(shape))
    return tuple(n for i, n in enumerate(shape) if i not in axes)


class Tensor:
    """A handle on a ``LazyNode``; every operation only extends the graph."""

    def __init__(
        self,
        data: ArrayLike,
        *,
        requires_grad: bool = False,
        dtype: Optional[object] = None,
        copy: bool = True,
    ) -> None:
        value = as_dtype(data, dtype) if dtype is not None else np.asarray(data)
        if requires_grad and not is_float(value.dtype):
            raise TypeError("only floating-point tensors can require gradients")
        self._node = LazyNode.leaf(value.copy() if copy else value, cache_native=copy)
        self.requires_grad = bool(requires_grad)
        self.grad: Optional[Tensor] = None
        self._is_leaf = True

    @classmethod
    def _wrap(cls, node: LazyNode, requires_grad: bool = False) -> "Tensor":
        tensor = cls.__new__(cls)
        tensor._node = node
        tensor.requires_grad = requires_grad and _GRAD_ENABLED
        tensor.grad = None
        tensor._is_leaf = False
        return tensor

    @classmethod
    def from_native(
        cls, value: object, *, backend: str, shape: Sequence[int], dtype: object
    ) -> "Tensor":
        """Wrap storage owned by a backend without copying it."""
        if not backend:
            raise ValueError("backend name cannot be empty")
        dims = tuple(int(size) for size in shape)
        if any(size < 0 for size in dims):
            raise ValueError("native tensor dimensions cannot be negative")
        tensor = cls._wrap(LazyNode.native_leaf(backend, value, dims, np.dtype(dtype)))
        tensor._is_leaf = True
        return tensor

    @classmethod
    def zeros(cls, shape: Sequence[int], *, dtype: object = np.float32) -> "Tensor":
        return cls(as_dtype(np.zeros(tuple(shape), dtype=np.float32), dtype), copy=False)

    @classmethod
    def ones(cls, shape: Sequence[int], *, dtype: object = np.float32) -> "Tensor":
        return cls(as_dtype(np.ones(tuple(shape), dtype=np.float32), dtype), copy=False)

    # -- metadata -------------------------------------------------------
    @property
    def shape(self) -> Tuple[int, ...]:
        return self._node.shape

    @property
    def ndim(self) -> int:
        return len(self._node.shape)

    @property
    def dtype(self) -> np.dtype:
        return self._node.dtype

    @property
    def T(self) -> "Tensor":
        if self.ndim != 2:
            raise ValueError("T is only defined for 2D tensors; use permute instead")
        return self.permute(1, 0)

    def numpy(self, compiler: Optional[str] = None) -> np.ndarray:
        return realize(self, compiler=compiler)[0]

    def item(self, compiler: Optional[str] = None) -> object:
        if self.shape != ():
            raise ValueError("item() requires a scalar tensor")
        return self.numpy(compiler).item()

    def detach(self) -> "Tensor":
        return Tensor._wrap(self._node)

    def assign(self, value: ArrayLike) -> None:
        """Replace a leaf's storage; graphs built earlier keep the old leaf."""
        if not self._is_leaf or self._node.value is None:
            raise RuntimeError("only leaf tensors can be assigned")
        replacement = as_dtype(value, self.dtype)
        if replacement.shape != self.shape:
            raise ValueError(f"expected shape {self.shape}, got {replacement.shape}")
        self._node = LazyNode.leaf(replacement.copy())

    def zero_grad(self) -> None:
        self.grad = None

    def backward(self, grad: Optional[ArrayLike] = None) -> None:
        raise NotImplementedError(
            "autograd belongs to the training path, which this build does not cover"
        )

    # -- elementwise ----------------------------------------------------
    def _coerce(self, other: Union["Tensor", ArrayLike]) -> "Tensor":
        return other if isinstance(other, Tensor) else Tensor(other, dtype=self.dtype)

    def _binary(self, other: Union["Tensor", ArrayLike], kind: str) -> "Tensor":
        right = self._coerce(other)
        shape = np.broadcast_shapes(self.shape, right.shape)
        dtype = result_type(self.dtype, right.dtype)
        node = LazyNode(Op.ELEMENTWISE, (self._node, right._node), kind, shape, dtype)
        return Tensor._wrap(node, self.requires_grad or right.requires_grad)

    def _unary(self, kind: str) -> "Tensor":
        node = LazyNode(Op.ELEMENTWISE, (self._node,), kind, self.shape, self.dtype)
        return Tensor._wrap(node, self.requires_grad)

    def __add__(self, other): return self._binary(other, "add")
    def __radd__(self, other): return self + other
    def __sub__(self, other): return self._binary(other, "sub")
    def __rsub__(self, other): return self._coerce(other) - self
    def __mul__(self, other): return self._binary(other, "mul")
    def __rmul__(self, other): return self * other
    def __truediv__(self, other): return self._binary(other, "div")
    def __rtruediv__(self, other): return self._coerce(other) / self
    def __neg__(self): return self._unary("neg")

    def equal(self, other: Union["Tensor", ArrayLike]) -> "Tensor":
        return self._binary(other, "equal")

    def exp(self) -> "Tensor": return self._unary("exp")
    def log(self) -> "Tensor": return self._unary("log")
    def relu(self) -> "Tensor": return self._unary("relu")
    def sqrt(self) -> "Tensor": return self._unary("sqrt")
    def step(self) -> "Tensor": return self._unary("step")

    # -- composites with lowering tags ------------------------------------
    def softmax(self, axis: int = -1) -> "Tensor":
        chosen = _axes(axis, self.ndim)[0]
        shifted = self - self.max(axis=axis, keepdims=True).detach()
        exponentials = shifted.exp()
        result = exponentials / exponentials.sum(axis=axis, keepdims=True)
        result._node.lowering = ("softmax", (self._node,), chosen)
        return result

    def log_softmax(self, axis: int = -1) -> "Tensor":
        chosen = _axes(axis, self.ndim)[0]
        shifted = self - self.max(axis=axis, keepdims=True).detach()
        result = shifted - shifted.exp().sum(axis=axis, keepdims=True).log()
        result._node.lowering = ("log_softmax", (self._node,), chosen)
        return result

    def layer_norm(self, weight: "Tensor", bias: "Tensor", epsilon: float = 1e-5) -> "Tensor":
        if self.ndim < 1:
            raise ValueError("layer_norm requires at least one dimension")
        expected = (self.shape[-1],)
        if weight.shape != expected or bias.shape != expected:
            raise ValueError(
                f"expected weight and bias shape {expected}, "
                f"got {weight.shape} and {bias.shape}"
            )
        if epsilon <= 0:
            raise ValueError("epsilon must be positive")
        centered = self - self.mean(axis=-1, keepdims=True)
        deviation = ((centered * centered).mean(axis=-1, keepdims=True) + epsilon).sqrt()
        result = centered / deviation * weight + bias
        result._node.lowering = (
            "layer_norm", (self._node, weight._node, bias._node), float(epsilon)
        )
        return result

    # -- shape ops --------------------------------------------------------
    def reshape(self, *shape: Union[int, Sequence[int]]) -> "Tensor":
        requested = (
            tuple(shape[0]) if len(shape) == 1 and not isinstance(shape[0], (int, np.integer))
            else tuple(shape)
        )
        dims = [int(size) for size in requested]
        total = int(np.prod(self.shape, dtype=np.int64))
        if dims.count(-1) > 1:
            raise ValueError("only one inferred dimension is allowed")
        if -1 in dims:
            known = int(np.prod([d for d in dims if d != -1], dtype=np.int64))
            if known == 0 or total % known:
                raise ValueError("shape is not compatible with tensor size")
            dims[dims.index(-1)] = total // known
        new_shape = tuple(dims)
        if int(np.prod(new_shape, dtype=np.int64)) != total:
            raise ValueError("shape is not compatible with tensor size")
        node = LazyNode(Op.RESHAPE, (self._node,), new_shape, new_shape, self.dtype)
        return Tensor._wrap(node, self.requires_grad)

    def permute(self, *axes: int) -> "Tensor":
        if len(axes) == 1 and not isinstance(axes[0], (int, np.integer)):
            axes = tuple(axes[0])
        order = tuple(int(a) for a in axes)
        if len(order) != self.ndim or set(order) != set(range(self.ndim)):
            raise ValueError(f"expected a permutation of {tuple(range(self.ndim))}")
        shape = tuple(self.shape[a] for a in order)
        node = LazyNode(Op.PERMUTE, (self._node,), order, shape, self.dtype)
        return Tensor._wrap(node, self.requires_grad)

    def transpose(self, dim0: int, dim1: int) -> "Tensor":
        first = dim0 + self.ndim if dim0 < 0 else dim0
        second = dim1 + self.ndim if dim1 < 0 else dim1
        if not (0 <= first < self.ndim and 0 <= second < self.ndim):
            raise ValueError(f"invalid transpose dimensions {dim0}, {dim1}")
        order = list(range(self.ndim))
        order[first], order[second] = order[second], order[first]
        return self.permute(*order)

    # -- contractions, selection, reductions --------------------------------
    def __matmul__(self, other: "Tensor") -> "Tensor":
        if not isinstance(other, Tensor):
            raise TypeError("matmul requires another Tensor")
        if self.ndim < 2 or other.ndim < 2:
            raise ValueError("matmul requires tensors with at least two dimensions")
        if self.shape[-1] != other.shape[-2]:
            raise ValueError(f"cannot multiply shapes {self.shape} and {other.shape}")
        batch = np.broadcast_shapes(self.shape[:-2], other.shape[:-2])
        shape = tuple(batch) + (self.shape[-2], other.shape[-1])
        dtype = result_type(self.dtype, other.dtype)
        node = LazyNode(Op.MATMUL, (self._node, other._node), None, shape, dtype)
        return Tensor._wrap(node, self.requires_grad or other.requires_grad)

    def gather(self, indices: "Tensor") -> "Tensor":
        """Rows of ``self`` selected by integer ``indices`` (axis 0)."""
        if not isinstance(indices, Tensor):
            raise TypeError("gather indices must be a Tensor")
        if not is_integer(indices.dtype):
            raise TypeError("gather indices must have an integer dtype")
        shape = indices.shape + self.shape[1:]
        node = LazyNode(Op.GATHER, (self._node, indices._node), None, shape, self.dtype)
        return Tensor._wrap(node, self.requires_grad)

    def sum(self, axis: Axis = None, keepdims: bool = False) -> "Tensor":
        axes = _axes(axis, self.ndim)
        node = LazyNode(
            Op.REDUCE, (self._node,), ("sum", axes, keepdims),
            _reduced(self.shape, axes, keepdims), self.dtype,
        )
        return Tensor._wrap(node, self.requires_grad)

    def mean(self, axis: Axis = None, keepdims: bool = False) -> "Tensor":
        axes = _axes(axis, self.ndim)
        count = int(np.prod([self.shape[a] for a in axes], dtype=np.int64))
        return self.sum(axis=axes, keepdims=keepdims) / count

    def max(self, axis: Axis = None, keepdims: bool = False) -> "Tensor":
        axes = _axes(axis, self.ndim)
        node = LazyNode(
            Op.REDUCE, (self._node,), ("max", axes, keepdims),
            _reduced(self.shape, axes, keepdims), self.dtype,
        )
        return Tensor._wrap(node, self.requires_grad)

    def __repr__(self) -> str:
        state = "leaf" if self._is_leaf else "lazy"
        return (
            f"Tensor(shape={self.shape}, dtype={self.dtype}, "
            f"requires_grad={self.requires_grad}, {state})"
        )


def realize(*tensors: Tensor, compiler: Optional[str] = None) -> Tuple[np.ndarray, ...]:
    return compile_graph(*tensors, compiler=compiler)()


def compile_graph(
    *tensors: Tensor,
    compiler: Optional[str] = None,
    dynamic_inputs: Sequence[Tensor] = (),
) -> CompiledProgram:
    if not tensors:
        raise ValueError("at least one tensor is required")
    selected = get_compiler(compiler)
    outputs = [tensor._node for tensor in tensors]
    if not dynamic_inputs:
        return selected.compile(outputs)
    return selected.compile(outputs, [tensor._node for tensor in dynamic_inputs])


__all__ = ["Tensor", "compile_graph", "no_grad", "realize", "BFLOAT16"]
