"""Host-side (numpy) helpers for the element formats of the C ABI.

bf16 values are carried on the host as uint16 bit patterns.  f32 -> bf16 uses the
reference rounding rule (src/utils/types.cpp:74-84: add 0x7FFF plus the kept LSB, shift),
so inputs built here are exactly the values the reference would have stored.
"""
import numpy as np

from .libllaisys import DataType

NUMPY_OF = {
    DataType.F32: np.float32,
    DataType.F16: np.float16,
    DataType.BF16: np.uint16,
    DataType.F64: np.float64,
    DataType.I8: np.int8,
    DataType.I16: np.int16,
    DataType.I32: np.int32,
    DataType.I64: np.int64,
    DataType.U8: np.uint8,
    DataType.U16: np.uint16,
    DataType.U32: np.uint32,
    DataType.U64: np.uint64,
    DataType.BOOL: np.bool_,
    DataType.BYTE: np.int8,
}


def f32_to_bf16(x) -> np.ndarray:
    """float32 array -> uint16 bf16 bits, reference round-half-even rule."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    """uint16 bf16 bits -> float32 (exact)."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_f32(arr: np.ndarray, dtype: DataType) -> np.ndarray:
    """Widens a host array holding `dtype` elements to float32."""
    if dtype == DataType.BF16:
        return bf16_to_f32(arr)
    return np.asarray(arr).astype(np.float32)


def from_f32(x, dtype: DataType) -> np.ndarray:
    """float32 values -> host array of `dtype` (bf16 via the reference rule)."""
    if dtype == DataType.BF16:
        return f32_to_bf16(x)
    if dtype == DataType.F32:
        return np.ascontiguousarray(x, dtype=np.float32)
    if dtype == DataType.F16:
        raise ValueError("f16 inputs: build them as np.float16 directly (exact values)")
    raise ValueError(f"not a float dtype: {dtype}")


def bf16_ulp_distance(a, b) -> np.ndarray:
    """|a - b| in units of bf16 ulps for finite bf16 bit patterns (monotone integer map)."""
    def key(u):
        u = np.asarray(u, dtype=np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - u, u)  # -0 and +0 both map to 0
    return np.abs(key(a) - key(b))
