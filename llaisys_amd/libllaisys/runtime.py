"""ctypes layout of LlaisysRuntimeAPI (include/llaisys/runtime.h).

Member order and signatures match the reference's
python/llaisys/libllaisys/runtime.py:6-48.
"""
from ctypes import CFUNCTYPE, POINTER, Structure, c_int, c_size_t, c_void_p

from .llaisys_types import llaisysDeviceType_t, llaisysMemcpyKind_t, llaisysStream_t

get_device_count_api = CFUNCTYPE(c_int)
set_device_api = CFUNCTYPE(None, c_int)
device_synchronize_api = CFUNCTYPE(None)
create_stream_api = CFUNCTYPE(llaisysStream_t)
destroy_stream_api = CFUNCTYPE(None, llaisysStream_t)
stream_synchronize_api = CFUNCTYPE(None, llaisysStream_t)
malloc_device_api = CFUNCTYPE(c_void_p, c_size_t)
free_device_api = CFUNCTYPE(None, c_void_p)
malloc_host_api = CFUNCTYPE(c_void_p, c_size_t)
free_host_api = CFUNCTYPE(None, c_void_p)
memcpy_sync_api = CFUNCTYPE(None, c_void_p, c_void_p, c_size_t, llaisysMemcpyKind_t)
memcpy_async_api = CFUNCTYPE(None, c_void_p, c_void_p, c_size_t, llaisysMemcpyKind_t,
                             llaisysStream_t)


class LlaisysRuntimeAPI(Structure):
    _fields_ = [
        ("get_device_count", get_device_count_api),
        ("set_device", set_device_api),
        ("device_synchronize", device_synchronize_api),
        ("create_stream", create_stream_api),
        ("destroy_stream", destroy_stream_api),
        ("stream_synchronize", stream_synchronize_api),
        ("malloc_device", malloc_device_api),
        ("free_device", free_device_api),
        ("malloc_host", malloc_host_api),
        ("free_host", free_host_api),
        ("memcpy_sync", memcpy_sync_api),
        ("memcpy_async", memcpy_async_api),
    ]


def load_runtime(lib):
    lib.llaisysGetRuntimeAPI.argtypes = [llaisysDeviceType_t]
    lib.llaisysGetRuntimeAPI.restype = POINTER(LlaisysRuntimeAPI)
    lib.llaisysSetContextRuntime.argtypes = [llaisysDeviceType_t, c_int]
    lib.llaisysSetContextRuntime.restype = None
    # additive entry points (absent from the reference library)
    if hasattr(lib, "llaisysGetContextStream"):
        lib.llaisysGetContextStream.argtypes = [llaisysDeviceType_t, c_int]
        lib.llaisysGetContextStream.restype = llaisysStream_t
    if hasattr(lib, "llaisysGraphBeginCapture"):
        lib.llaisysGraphBeginCapture.argtypes = [llaisysDeviceType_t, c_int]
        lib.llaisysGraphBeginCapture.restype = None
        lib.llaisysGraphEndCapture.argtypes = [llaisysDeviceType_t, c_int]
        lib.llaisysGraphEndCapture.restype = c_void_p
        lib.llaisysGraphLaunch.argtypes = [c_void_p]
        lib.llaisysGraphLaunch.restype = None
        lib.llaisysGraphDestroy.argtypes = [c_void_p]
        lib.llaisysGraphDestroy.restype = None
    if hasattr(lib, "llaisysTakeDeviceError"):
        lib.llaisysTakeDeviceError.argtypes = [llaisysDeviceType_t, c_int]
        lib.llaisysTakeDeviceError.restype = c_int
