"""RuntimeAPI: the device runtime table as Python methods.

Same methods as the reference's python/llaisys/runtime.py:6-68 (the reference prints on
every free_device, :37; this one does not).
"""
from . import libllaisys
from .libllaisys import LIB_LLAISYS


class RuntimeAPI:
    def __init__(self, device_type: libllaisys.DeviceType, lib=None):
        self._lib = lib if lib is not None else LIB_LLAISYS
        self._api = self._lib.llaisysGetRuntimeAPI(libllaisys.llaisysDeviceType_t(device_type))

    def get_device_count(self) -> int:
        return self._api.contents.get_device_count()

    def set_device(self, device_id: int) -> None:
        self._api.contents.set_device(device_id)

    def device_synchronize(self) -> None:
        self._api.contents.device_synchronize()

    def create_stream(self):
        return self._api.contents.create_stream()

    def destroy_stream(self, stream) -> None:
        self._api.contents.destroy_stream(stream)

    def stream_synchronize(self, stream) -> None:
        self._api.contents.stream_synchronize(stream)

    def malloc_device(self, size: int):
        return self._api.contents.malloc_device(size)

    def free_device(self, ptr) -> None:
        self._api.contents.free_device(ptr)

    def malloc_host(self, size: int):
        return self._api.contents.malloc_host(size)

    def free_host(self, ptr) -> None:
        self._api.contents.free_host(ptr)

    def memcpy_sync(self, dst, src, size: int, kind: libllaisys.MemcpyKind) -> None:
        self._api.contents.memcpy_sync(dst, src, size, libllaisys.llaisysMemcpyKind_t(kind))

    def memcpy_async(self, dst, src, size: int, kind: libllaisys.MemcpyKind, stream) -> None:
        self._api.contents.memcpy_async(dst, src, size, libllaisys.llaisysMemcpyKind_t(kind),
                                        stream)


def context_stream(device_type=libllaisys.DeviceType.AMD, device_id: int = 0, lib=None) -> int:
    """Raw stream handle the ops of (device_type, device_id) run on (llaisysGetContextStream)."""
    lib = lib if lib is not None else LIB_LLAISYS
    return lib.llaisysGetContextStream(int(device_type), int(device_id)) or 0


def take_device_error(device_type=libllaisys.DeviceType.AMD, device_id: int = 0, lib=None) -> int:
    """Waits for the context stream and returns / clears the sticky device error code."""
    lib = lib if lib is not None else LIB_LLAISYS
    return int(lib.llaisysTakeDeviceError(int(device_type), int(device_id)))


class Graph:
    """HIP graph of the ops issued between capture() and end() on (device_type, device_id).

        g = Graph.capture()          # ops below are recorded, not run
        Ops.swiglu(out, gate, up)
        g.end()
        g.launch()                   # replays on the context stream
    """

    def __init__(self, device_type, device_id, lib):
        self._lib, self._dt, self._id, self._g = lib, int(device_type), int(device_id), None

    @classmethod
    def capture(cls, device_type=libllaisys.DeviceType.AMD, device_id: int = 0, lib=None):
        g = cls(device_type, device_id, lib if lib is not None else LIB_LLAISYS)
        g._lib.llaisysGraphBeginCapture(g._dt, g._id)
        return g

    def end(self) -> "Graph":
        self._g = self._lib.llaisysGraphEndCapture(self._dt, self._id)
        return self

    def launch(self) -> None:
        self._lib.llaisysGraphLaunch(self._g)

    def __del__(self):
        if getattr(self, "_g", None):
            self._lib.llaisysGraphDestroy(self._g)
            self._g = None
