"""llaisys_amd: MI355X (gfx950) build of the LLAISYS per-layer ops behind the LLAISYS C ABI.

Same top-level names as the reference package python/llaisys/__init__.py:1-20
(RuntimeAPI, DeviceType, DataType, MemcpyKind, Stream, Tensor, Ops); the model driver is
not part of this package.
"""
from .libllaisys import DataType, DeviceType, MemcpyKind
from .libllaisys import llaisysStream_t as Stream
from .ops import Ops
from .runtime import Graph, RuntimeAPI, context_stream, take_device_error
from .tensor import Tensor

__all__ = [
    "RuntimeAPI",
    "DeviceType",
    "DataType",
    "MemcpyKind",
    "Stream",
    "Tensor",
    "Ops",
    "Graph",
    "context_stream",
    "take_device_error",
]
