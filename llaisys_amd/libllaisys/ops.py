"""ctypes signatures of the op entry points (include/llaisys/ops.h).

The nine reference entry points have the argtypes of the reference's
python/llaisys/libllaisys/ops.py:4-36; the additive ones are bound when present, so the
same loader also binds the reference library (used to write golden vectors).
"""
from ctypes import c_float, c_int64, c_size_t, c_uint8, c_uint64

from .tensor import llaisysTensor_t

T = llaisysTensor_t

REFERENCE_OPS = {
    "llaisysAdd": [T, T, T],
    "llaisysArgmax": [T, T, T],
    "llaisysEmbedding": [T, T, T],
    "llaisysLinear": [T, T, T, T],
    "llaisysRearrange": [T, T],
    "llaisysRmsNorm": [T, T, T, c_float],
    "llaisysROPE": [T, T, T, c_float],
    "llaisysSelfAttention": [T, T, T, T, c_float],
    "llaisysSwiGLU": [T, T, T],
}

ADDED_OPS = {
    "llaisysAddRmsNorm": [T, T, T, T, T, c_float],
    "llaisysROPEQK": [T, T, T, T, T, c_float],
    "llaisysROPEKVAppendInt8": [T, T, T, T, T, c_float, T, T, T, T, c_size_t],
    "llaisysArgmaxRows": [T, T, T],
    "llaisysQuantizeInt8": [T, T, T],
    "llaisysDequantizeInt8": [T, T, T],
    "llaisysKVAppendInt8": [T, T, T, c_size_t],
    "llaisysKVAppendInt8Pair": [T, T, T, T, T, T, c_size_t],
    "llaisysDequantizeInt8Pair": [T, T, T, T, T, T],
    "llaisysSelfAttentionInt8KV": [T, T, T, T, T, T, c_float],
    "llaisysSelfAttentionInt8KVNoAlloc": [T, T, T, T, T, T, c_float],
    "llaisysCast": [T, T],
    "llaisysLinearW8A16": [T, T, T, T, T],
    "llaisysRandomSample": [T, T, c_float, c_int64, c_float, c_uint64],
    "llaisysRmsNormLinear": [T, T, T, T, T, c_float, T, T, T, c_uint8],
}


def load_ops(lib):
    for name, args in REFERENCE_OPS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None
    for name, args in ADDED_OPS.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None
