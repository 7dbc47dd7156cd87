"""Tensor: owning Python handle of an llaisysTensor_t.

Same methods as the reference's python/llaisys/tensor.py:14-97, plus numpy helpers
(from_numpy / numpy) used by tests and benchmarks.  `lib` selects the library the handle
belongs to (default: this package's libllaisys.so).
"""
from ctypes import c_int, c_size_t, c_ssize_t, c_void_p
from typing import Sequence, Tuple

import numpy as np

from .hostfmt import NUMPY_OF
from .libllaisys import (LIB_LLAISYS, DataType, DeviceType, MemcpyKind, llaisysDataType_t,
                         llaisysDeviceType_t, llaisysTensor_t)


class Tensor:
    def __init__(self, shape: Sequence[int] = None, dtype: DataType = DataType.F32,
                 device: DeviceType = DeviceType.CPU, device_id: int = 0,
                 tensor: llaisysTensor_t = None, lib=None):
        self._lib = lib if lib is not None else LIB_LLAISYS
        if tensor:
            self._tensor = tensor
        else:
            ndim = 0 if shape is None else len(shape)
            dims = None if shape is None else (c_size_t * ndim)(*shape)
            self._tensor = self._lib.tensorCreate(dims, c_size_t(ndim), llaisysDataType_t(dtype),
                                                  llaisysDeviceType_t(device), c_int(device_id))

    def __del__(self):
        if getattr(self, "_tensor", None) is not None:
            self._lib.tensorDestroy(self._tensor)
            self._tensor = None

    # ---- reference API --------------------------------------------------------------
    def shape(self) -> Tuple[int, ...]:
        buf = (c_size_t * self.ndim())()
        self._lib.tensorGetShape(self._tensor, buf)
        return tuple(buf)

    def strides(self) -> Tuple[int, ...]:
        buf = (c_ssize_t * self.ndim())()
        self._lib.tensorGetStrides(self._tensor, buf)
        return tuple(buf)

    def ndim(self) -> int:
        return int(self._lib.tensorGetNdim(self._tensor))

    def dtype(self) -> DataType:
        return DataType(self._lib.tensorGetDataType(self._tensor))

    def device_type(self) -> DeviceType:
        return DeviceType(self._lib.tensorGetDeviceType(self._tensor))

    def device_id(self) -> int:
        return int(self._lib.tensorGetDeviceId(self._tensor))

    def data_ptr(self) -> c_void_p:
        return self._lib.tensorGetData(self._tensor)

    def lib_tensor(self) -> llaisysTensor_t:
        return self._tensor

    def debug(self):
        self._lib.tensorDebug(self._tensor)

    def __repr__(self):
        return (f"<Tensor shape={self.shape()}, dtype={self.dtype().name}, "
                f"device={self.device_type().name}:{self.device_id()}>")

    def load(self, data: c_void_p):
        self._lib.tensorLoad(self._tensor, data)

    def is_contiguous(self) -> bool:
        return bool(self._lib.tensorIsContiguous(self._tensor))

    def view(self, *shape: int) -> "Tensor":
        dims = (c_size_t * len(shape))(*shape)
        return Tensor(tensor=self._lib.tensorView(self._tensor, dims, c_size_t(len(shape))),
                      lib=self._lib)

    def permute(self, *perm: int) -> "Tensor":
        assert len(perm) == self.ndim()
        order = (c_size_t * len(perm))(*perm)
        return Tensor(tensor=self._lib.tensorPermute(self._tensor, order), lib=self._lib)

    def slice(self, dim: int, start: int, end: int) -> "Tensor":
        return Tensor(tensor=self._lib.tensorSlice(self._tensor, c_size_t(dim), c_size_t(start),
                                                   c_size_t(end)), lib=self._lib)

    def contiguous(self) -> "Tensor":
        """This tensor when contiguous (shared storage), else a contiguous copy on the same
        device (reference Tensor::contiguous, src/tensor/tensor.hpp:55)."""
        return Tensor(tensor=self._lib.tensorContiguous(self._tensor), lib=self._lib)

    def reshape(self, *shape: int) -> "Tensor":
        """A view when contiguous, else a view of contiguous() (reference tensor.hpp:56)."""
        dims = (c_size_t * len(shape))(*shape)
        return Tensor(tensor=self._lib.tensorReshape(self._tensor, dims, c_size_t(len(shape))),
                      lib=self._lib)

    def to(self, device: "DeviceType", device_id: int = -1) -> "Tensor":
        """This tensor when already on (device, device_id), else a contiguous copy there
        (reference Tensor::to, tensor.hpp:57).  Synchronous."""
        return Tensor(tensor=self._lib.tensorTo(self._tensor, device, c_int(device_id)), lib=self._lib)

    # ---- numpy helpers --------------------------------------------------------------
    def numel(self) -> int:
        return int(np.prod(self.shape(), dtype=np.int64))

    @classmethod
    def from_numpy(cls, arr: np.ndarray, dtype: DataType = None,
                   device: DeviceType = DeviceType.AMD, device_id: int = 0, lib=None) -> "Tensor":
        """New contiguous tensor holding a copy of `arr` (bf16 given as uint16 bits)."""
        if dtype is None:
            dtype = {np.dtype(v): k for k, v in NUMPY_OF.items()
                     if k not in (DataType.BF16, DataType.BYTE)}[arr.dtype]
        host = np.ascontiguousarray(arr, dtype=NUMPY_OF[dtype])
        t = cls(host.shape, dtype, device, device_id, lib=lib)
        if host.size:
            t.load(host.ctypes.data_as(c_void_p))
        return t

    def numpy(self) -> np.ndarray:
        """Synchronous copy of a contiguous tensor to a new host array."""
        if not self.is_contiguous():
            raise ValueError("numpy() needs a contiguous tensor")
        out = np.empty(self.shape(), dtype=NUMPY_OF[self.dtype()])
        if out.size:
            from .runtime import RuntimeAPI
            kind = MemcpyKind.D2H if self.device_type() != DeviceType.CPU else MemcpyKind.H2H
            RuntimeAPI(self.device_type(), lib=self._lib).memcpy_sync(
                out.ctypes.data_as(c_void_p), self.data_ptr(), out.nbytes, kind)
        return out
