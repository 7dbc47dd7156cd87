"""ctypes signatures of the tensor entry points (include/llaisys/tensor.h).

Same argtypes as the reference's python/llaisys/libllaisys/tensor.py:8-78.
"""
from ctypes import POINTER, c_int, c_size_t, c_ssize_t, c_uint8, c_void_p

from .llaisys_types import llaisysDataType_t, llaisysDeviceType_t

llaisysTensor_t = c_void_p


def load_tensor(lib):
    sigs = {
        "tensorCreate": ([POINTER(c_size_t), c_size_t, llaisysDataType_t, llaisysDeviceType_t,
                          c_int], llaisysTensor_t),
        "tensorDestroy": ([llaisysTensor_t], None),
        "tensorGetData": ([llaisysTensor_t], c_void_p),
        "tensorGetNdim": ([llaisysTensor_t], c_size_t),
        "tensorGetShape": ([llaisysTensor_t, POINTER(c_size_t)], None),
        "tensorGetStrides": ([llaisysTensor_t, POINTER(c_ssize_t)], None),
        "tensorGetDataType": ([llaisysTensor_t], llaisysDataType_t),
        "tensorGetDeviceType": ([llaisysTensor_t], llaisysDeviceType_t),
        "tensorGetDeviceId": ([llaisysTensor_t], c_int),
        "tensorDebug": ([llaisysTensor_t], None),
        "tensorIsContiguous": ([llaisysTensor_t], c_uint8),
        "tensorLoad": ([llaisysTensor_t, c_void_p], None),
        "tensorView": ([llaisysTensor_t, POINTER(c_size_t), c_size_t], llaisysTensor_t),
        "tensorPermute": ([llaisysTensor_t, POINTER(c_size_t)], llaisysTensor_t),
        "tensorSlice": ([llaisysTensor_t, c_size_t, c_size_t, c_size_t], llaisysTensor_t),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    # additive entry points (bound when present, so the reference library also loads)
    added = {
        "tensorContiguous": ([llaisysTensor_t], llaisysTensor_t),
        "tensorReshape": ([llaisysTensor_t, POINTER(c_size_t), c_size_t], llaisysTensor_t),
        "tensorTo": ([llaisysTensor_t, llaisysDeviceType_t, c_int], llaisysTensor_t),
    }
    for name, (args, res) in added.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
