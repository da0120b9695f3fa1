"""Device backends: the ``DeviceBackend`` contract and ``MI355XBackend``, the ROCm backend
built on ``libmoe_mi355x.so``.

Contract and error behaviour follow offload_runtime/backends/base.py:9-77 and
offload_runtime/backends/rocm_backend.py:33-119 (name ``"rocm"``, non-blocking streams,
events created without timing, ``ValueError`` for undersized or read-only host views,
``RuntimeError`` for failed HIP calls).  The ROCm backend reaches HIP through the C ABI
of this package instead of hip-python.
"""
from __future__ import annotations

import ctypes
from abc import ABC, abstractmethod
from typing import Any

from . import _lib
from .types import DeviceBuffer, HostBuffer


class DeviceBackend(ABC):
    """Vendor device API adapter used by the runtime and the executors."""

    name: str

    @abstractmethod
    def create_stream(self, purpose: str) -> Any: ...

    @abstractmethod
    def destroy_stream(self, stream: Any) -> None: ...

    @abstractmethod
    def alloc_device(self, nbytes: int) -> DeviceBuffer: ...

    @abstractmethod
    def free_device(self, buf: DeviceBuffer) -> None: ...

    @property
    def supports_pinned_host(self) -> bool:
        return False

    @property
    def supports_peer_to_peer(self) -> bool:
        return False

    @property
    def supports_graph_capture(self) -> bool:
        return False

    def alloc_pinned_host(self, nbytes: int) -> HostBuffer:
        raise NotImplementedError(f"{self.name} does not support pinned host memory")

    def free_pinned_host(self, buf: HostBuffer) -> None:
        raise NotImplementedError(f"{self.name} does not support pinned host memory")

    @abstractmethod
    def copy_h2d_async(self, dst: DeviceBuffer, src: HostBuffer, stream: Any) -> None: ...

    @abstractmethod
    def copy_d2h_async(self, dst: HostBuffer, src: DeviceBuffer, stream: Any) -> None: ...

    @abstractmethod
    def record_event(self, stream: Any) -> Any: ...

    @abstractmethod
    def destroy_event(self, event: Any) -> None: ...

    @abstractmethod
    def wait_event(self, stream: Any, event: Any) -> None: ...

    @abstractmethod
    def synchronize_stream(self, stream: Any) -> None: ...


def _view_address(view: memoryview) -> int:
    """Address of a host view; async copies need a writable, contiguous view
    (rocm_backend.py:27-30 raises ValueError for read-only views in both directions)."""
    if view.readonly:
        raise ValueError("HostBuffer.view must be writable for async hipMemcpyAsync.")
    if not view.c_contiguous:
        raise ValueError("HostBuffer.view must be C-contiguous")
    if view.nbytes == 0:
        return 0
    return ctypes.addressof(ctypes.c_char.from_buffer(view.cast("B")))


class MI355XBackend(DeviceBackend):
    """ROCm backend for one MI355X (gfx950) device over ``libmoe_mi355x.so``."""

    name = "rocm"

    def __init__(self, device_id: int = 0) -> None:
        self._lib = _lib.load()
        self.device_id = device_id
        _lib.check(self._lib.mx_set_device(device_id), "hipSetDevice")
        self._pinned: dict[int, int] = {}  # address -> nbytes

    # -- capabilities (rocm_backend.py:51-61) --
    @property
    def supports_pinned_host(self) -> bool:
        return True

    @property
    def supports_peer_to_peer(self) -> bool:
        return True

    @property
    def supports_graph_capture(self) -> bool:
        return True

    # -- pinned host memory --
    def alloc_pinned_host(self, nbytes: int) -> HostBuffer:
        ptr = ctypes.c_void_p()
        _lib.check(self._lib.mx_host_malloc(ctypes.byref(ptr), nbytes), "hipHostMalloc")
        addr = int(ptr.value)
        arr = (ctypes.c_byte * nbytes).from_address(addr)
        self._pinned[addr] = nbytes
        return HostBuffer(view=memoryview(arr).cast("B"), pinned=True)

    def free_pinned_host(self, buf: HostBuffer) -> None:
        addr = _view_address(buf.view)
        self._pinned.pop(addr, None)
        _lib.check(self._lib.mx_host_free(addr), "hipHostFree")

    # -- streams --
    def create_stream(self, purpose: str) -> Any:
        s = ctypes.c_void_p()
        _lib.check(self._lib.mx_stream_create(ctypes.byref(s), 1), "hipStreamCreateWithFlags")
        return int(s.value)

    def destroy_stream(self, stream: Any) -> None:
        _lib.check(self._lib.mx_stream_destroy(stream), "hipStreamDestroy")

    # -- device memory --
    def alloc_device(self, nbytes: int) -> DeviceBuffer:
        p = ctypes.c_void_p()
        _lib.check(self._lib.mx_malloc(ctypes.byref(p), nbytes), "hipMalloc")
        return DeviceBuffer(handle=int(p.value), nbytes=nbytes, backend=self.name)

    def free_device(self, buf: DeviceBuffer) -> None:
        _lib.check(self._lib.mx_free(buf.handle), "hipFree")

    # -- copies (rocm_backend.py:88-104) --
    def copy_h2d_async(self, dst: DeviceBuffer, src: HostBuffer, stream: Any) -> None:
        if src.nbytes < dst.nbytes:
            raise ValueError(
                f"Host buffer ({src.nbytes}B) smaller than device buffer ({dst.nbytes}B)")
        addr = _view_address(src.view)
        _lib.check(self._lib.mx_memcpy_h2d_async(dst.handle, addr, dst.nbytes, stream),
                   "hipMemcpyAsync(H2D)")

    def copy_d2h_async(self, dst: HostBuffer, src: DeviceBuffer, stream: Any) -> None:
        if dst.nbytes < src.nbytes:
            raise ValueError(
                f"Host buffer ({dst.nbytes}B) smaller than device buffer ({src.nbytes}B)")
        addr = _view_address(dst.view)
        _lib.check(self._lib.mx_memcpy_d2h_async(addr, src.handle, src.nbytes, stream),
                   "hipMemcpyAsync(D2H)")

    # -- events (rocm_backend.py:106-116) --
    def record_event(self, stream: Any) -> Any:
        ev = ctypes.c_void_p()
        _lib.check(self._lib.mx_event_create(ctypes.byref(ev), 0), "hipEventCreateWithFlags")
        _lib.check(self._lib.mx_event_record(ev, stream), "hipEventRecord")
        return int(ev.value)

    def destroy_event(self, event: Any) -> None:
        _lib.check(self._lib.mx_event_destroy(event), "hipEventDestroy")

    def wait_event(self, stream: Any, event: Any) -> None:
        _lib.check(self._lib.mx_event_wait(stream, event), "hipStreamWaitEvent")

    def synchronize_stream(self, stream: Any) -> None:
        _lib.check(self._lib.mx_stream_sync(stream), "hipStreamSynchronize")

    # -- extras used by the MoE executors and the runtime --
    def copy_h2d_ptr_async(self, dst: int, src_addr: int, nbytes: int, stream: Any) -> None:
        _lib.check(self._lib.mx_memcpy_h2d_async(dst, src_addr, nbytes, stream),
                   "hipMemcpyAsync(H2D)")

    def copy_d2h_ptr_async(self, dst_addr: int, src: int, nbytes: int, stream: Any) -> None:
        _lib.check(self._lib.mx_memcpy_d2h_async(dst_addr, src, nbytes, stream),
                   "hipMemcpyAsync(D2H)")

    def create_timing_event(self) -> int:
        ev = ctypes.c_void_p()
        _lib.check(self._lib.mx_event_create(ctypes.byref(ev), 1), "hipEventCreate")
        return int(ev.value)

    def record(self, event: int, stream: Any) -> None:
        _lib.check(self._lib.mx_event_record(event, stream), "hipEventRecord")

    def elapsed_ms(self, start: int, end: int) -> float:
        ms = ctypes.c_float()
        _lib.check(self._lib.mx_event_elapsed_ms(ctypes.byref(ms), start, end),
                   "hipEventElapsedTime")
        return float(ms.value)

    def event_synchronize(self, event: int) -> None:
        _lib.check(self._lib.mx_event_sync(event), "hipEventSynchronize")

    def event_done(self, event: int) -> bool:
        done = ctypes.c_int32(0)
        _lib.check(self._lib.mx_event_query(event, ctypes.byref(done)), "hipEventQuery")
        return bool(done.value)


# Name used by the reference package for its ROCm adapter.
ROCmBackend = MI355XBackend


def detect_backend(device_id: int = 0) -> DeviceBackend:
    """The MI355X backend (the ROCm entry of offload_runtime/backends/__init__.py:22-31).

    There is no CPU fallback: the MoE step only runs in the HIP library, so a missing
    library or device raises ``RuntimeError`` instead of handing back a host stand-in."""
    lib = _lib.load()
    n = ctypes.c_int32(0)
    rc = lib.mx_get_device_count(ctypes.byref(n))
    if rc != 0 or n.value <= device_id:
        raise RuntimeError(f"no ROCm device {device_id} (hipGetDeviceCount status {rc}, "
                           f"{n.value} devices)")
    return MI355XBackend(device_id)
