"""Element types understood by the IR and the ``hip`` plugin.

NumPy has no bfloat16 and ``ml_dtypes`` is not a dependency here, so bf16
tensors use a two-byte structured dtype as their marker (``BFLOAT16``).  Its
storage is the upper half of an IEEE float32; conversion from float32 rounds
to nearest, ties to even, and NaN stays NaN.

The reference maps bf16 natives to ``ml_dtypes.bfloat16``
(chomikgrad/mlx_backend.py:67-75); a device adapter here reports ``BFLOAT16``
instead.
"""

from __future__ import annotations

import numpy as np

BFLOAT16 = np.dtype([("bfloat16", "<u2")])

# Integer codes shared with the C ABI (include/chomik_hip.h, CHIP_DTYPE_*).
DT_F32 = 0
DT_F16 = 1
DT_BF16 = 2
DT_I32 = 3
DT_I64 = 4

_CODES = {
    np.dtype(np.float32).str: DT_F32,
    np.dtype(np.float16).str: DT_F16,
    BFLOAT16.str: DT_BF16,
    np.dtype(np.int32).str: DT_I32,
    np.dtype(np.int64).str: DT_I64,
}


def is_bf16(dtype: object) -> bool:
    return np.dtype(dtype) == BFLOAT16


def is_float(dtype: object) -> bool:
    dtype = np.dtype(dtype)
    return dtype == BFLOAT16 or np.issubdtype(dtype, np.floating)


def is_integer(dtype: object) -> bool:
    dtype = np.dtype(dtype)
    return dtype != BFLOAT16 and np.issubdtype(dtype, np.integer)


def dtype_code(dtype: object) -> int:
    """Map a NumPy dtype to the ABI code, or raise ``TypeError``."""
    key = np.dtype(dtype).str
    try:
        return _CODES[key]
    except KeyError as error:
        raise TypeError(
            f"the hip backend does not support dtype {np.dtype(dtype)}; "
            "use float32, float16, bfloat16, int32 or int64"
        ) from error


def float32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 bit patterns (nearest, ties to even)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    upper = bits >> np.uint32(16)
    lsb = upper & np.uint32(1)
    rounded = (bits + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    nan = (bits & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    quiet = (upper | np.uint32(0x40)) & np.uint32(0xFFFF)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def to_bf16(values: object) -> np.ndarray:
    """Convert numbers (any float/int array-like) to a ``BFLOAT16`` array."""
    array = np.asarray(values)
    if array.dtype == BFLOAT16:
        return array
    bits = float32_to_bf16_bits(array.astype(np.float32))
    return bits.view(BFLOAT16).reshape(array.shape)


def bf16_to_float32(values: np.ndarray) -> np.ndarray:
    array = np.asarray(values)
    if array.dtype != BFLOAT16:
        raise TypeError("expected a bfloat16 array")
    bits = np.ascontiguousarray(array).view(np.uint16).astype(np.uint32)
    return (bits << np.uint32(16)).view(np.float32).reshape(array.shape)


def as_dtype(values: object, dtype: object) -> np.ndarray:
    """``np.asarray(values, dtype)`` that also understands ``BFLOAT16``."""
    dtype = np.dtype(dtype)
    if dtype == BFLOAT16:
        return to_bf16(values)
    array = np.asarray(values)
    if array.dtype == BFLOAT16:
        array = bf16_to_float32(array)
    return np.asarray(array, dtype=dtype)


def result_type(left: object, right: object) -> np.dtype:
    """NumPy promotion extended with ``BFLOAT16``.

    bf16 with bf16 stays bf16; bf16 with a wider float promotes to that float
    (float16 is not wider: bf16 with float16 gives float32, as in ml_dtypes).
    """
    left, right = np.dtype(left), np.dtype(right)
    if left != BFLOAT16 and right != BFLOAT16:
        return np.result_type(left, right)
    if left == right:
        return BFLOAT16
    other = right if left == BFLOAT16 else left
    if other in (np.dtype(np.float32), np.dtype(np.float64)):
        return other
    return np.dtype(np.float32)


def dtype_name(dtype: object) -> str:
    dtype = np.dtype(dtype)
    return "bfloat16" if dtype == BFLOAT16 else dtype.name
