"""Runtime table wrapper (reference: python/llaisys/runtime.py:6-68)."""
from ctypes import c_void_p

from .libllaisys import (
    LIB_LLAISYS,
    DeviceType,
    MemcpyKind,
    check_last_error,
    llaisysDeviceType_t,
    llaisysMemcpyKind_t,
    llaisysStream_t,
)


class RuntimeAPI:
    def __init__(self, device_type: DeviceType):
        self._api = LIB_LLAISYS.llaisysGetRuntimeAPI(llaisysDeviceType_t(device_type))
        check_last_error()

    def get_device_count(self) -> int:
        return self._api.contents.get_device_count()

    def set_device(self, device_id: int) -> None:
        self._api.contents.set_device(device_id)

    def device_synchronize(self) -> None:
        self._api.contents.device_synchronize()

    def create_stream(self) -> llaisysStream_t:
        return self._api.contents.create_stream()

    def destroy_stream(self, stream: llaisysStream_t) -> None:
        self._api.contents.destroy_stream(stream)

    def stream_synchronize(self, stream: llaisysStream_t) -> None:
        self._api.contents.stream_synchronize(stream)

    def malloc_device(self, size: int) -> c_void_p:
        return self._api.contents.malloc_device(size)

    def free_device(self, ptr: c_void_p) -> None:
        self._api.contents.free_device(ptr)

    def malloc_host(self, size: int) -> c_void_p:
        return self._api.contents.malloc_host(size)

    def free_host(self, ptr: c_void_p) -> None:
        self._api.contents.free_host(ptr)

    def memcpy_sync(self, dst: c_void_p, src: c_void_p, size: int, kind: MemcpyKind) -> None:
        self._api.contents.memcpy_sync(dst, src, size, llaisysMemcpyKind_t(kind))

    def memcpy_async(self, dst: c_void_p, src: c_void_p, size: int, kind: MemcpyKind, stream: llaisysStream_t) -> None:
        self._api.contents.memcpy_async(dst, src, size, llaisysMemcpyKind_t(kind), stream)


def set_context_runtime(device: DeviceType, device_id: int = 0) -> None:
    """Activate (device, id) for the calling thread (llaisysSetContextRuntime)."""
    LIB_LLAISYS.llaisysSetContextRuntime(llaisysDeviceType_t(device), device_id)
    check_last_error()


def context_stream() -> int:
    """The HIP stream the calling thread's active runtime launches kernels on."""
    s = LIB_LLAISYS.llaisysGetContextStream()
    check_last_error()
    return int(s or 0)


def set_context_stream(stream: int) -> None:
    """Launch subsequent ops of this thread on `stream` (0 restores the runtime's own)."""
    LIB_LLAISYS.llaisysSetContextStream(c_void_p(stream or None))
    check_last_error()


def device_error_flags() -> int:
    """Kernel-side error bits since the last call (1 bad block id, 2 context too long); syncs."""
    f = LIB_LLAISYS.llaisysGetDeviceErrorFlags()
    check_last_error()
    return int(f)
