"""Loads libllaisys.so (the MI355X build) and binds its C ABI with ctypes.

Mirrors the reference loader python/llaisys/libllaisys/__init__.py:18-42.  The library
must have been built (`python -c "import __graft_entry__ as g; g.build()"` or
`make -C llaisys_amd/csrc`); a missing library is an error, there is no fallback.
"""
import ctypes
import os
from pathlib import Path

from .llaisys_types import (DataType, DeviceType, MemcpyKind, llaisysDataType_t,
                            llaisysDeviceType_t, llaisysMemcpyKind_t, llaisysStream_t)
from .ops import load_ops
from .runtime import LlaisysRuntimeAPI, load_runtime
from .tensor import llaisysTensor_t, load_tensor

LIB_PATH = Path(__file__).parent / "libllaisys.so"


def bind(lib):
    """Sets the argtypes / restypes of every LLAISYS entry point `lib` exports."""
    load_runtime(lib)
    load_tensor(lib)
    load_ops(lib)
    return lib


def load_shared_library(path=None):
    path = Path(path) if path is not None else LIB_PATH
    if not os.path.isfile(path):
        raise FileNotFoundError(
            f"Shared library not found: {path} (build it with make -C llaisys_amd/csrc)")
    return bind(ctypes.CDLL(str(path)))


LIB_LLAISYS = load_shared_library()

__all__ = [
    "LIB_LLAISYS",
    "LIB_PATH",
    "bind",
    "load_shared_library",
    "LlaisysRuntimeAPI",
    "llaisysStream_t",
    "llaisysTensor_t",
    "llaisysDataType_t",
    "DataType",
    "llaisysDeviceType_t",
    "DeviceType",
    "llaisysMemcpyKind_t",
    "MemcpyKind",
]
