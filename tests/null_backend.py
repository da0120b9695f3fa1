"""CPU stand-in for a device backend, used by the CPU tests of the runtime, the pools and
the executors' host logic: device buffers are bytearrays keyed by ``id``, copies are
synchronous, streams and events are opaque tokens.  It follows the behaviour of
offload_runtime/backends/null_backend.py:9-76, which the reference's own tests rely on
(``backend._buffers`` to check frees, tests/test_runtime.py:145-157).  Test-only: the
product package has no CPU fallback.
"""
from __future__ import annotations

from typing import Any

from moe_mi355x.backends import DeviceBackend
from moe_mi355x.types import DeviceBuffer, HostBuffer


class NullBackend(DeviceBackend):
    """CPU stand-in: device buffers are bytearrays, copies are synchronous, streams and
    events are opaque tokens.  Used by the CPU tests of the runtime and pools
    (behaviour of offload_runtime/backends/null_backend.py:9-76)."""

    name = "null"

    def __init__(self) -> None:
        self._buffers: dict[int, bytearray] = {}
        self._pinned: set[int] = set()

    @property
    def supports_pinned_host(self) -> bool:
        return True

    def alloc_pinned_host(self, nbytes: int) -> HostBuffer:
        buf = bytearray(nbytes)
        self._pinned.add(id(buf))
        return HostBuffer(view=memoryview(buf), pinned=True)

    def free_pinned_host(self, buf: HostBuffer) -> None:
        self._pinned.discard(id(buf.view.obj))

    def create_stream(self, purpose: str) -> Any:
        return object()

    def destroy_stream(self, stream: Any) -> None:
        return None

    def alloc_device(self, nbytes: int) -> DeviceBuffer:
        buf = bytearray(nbytes)
        self._buffers[id(buf)] = buf
        return DeviceBuffer(handle=id(buf), nbytes=nbytes, backend=self.name)

    def free_device(self, buf: DeviceBuffer) -> None:
        self._buffers.pop(int(buf.handle), None)

    def copy_h2d_async(self, dst: DeviceBuffer, src: HostBuffer, stream: Any) -> None:
        target = self._buffers[int(dst.handle)]
        data = src.view.tobytes()
        target[: len(data)] = data

    def copy_d2h_async(self, dst: HostBuffer, src: DeviceBuffer, stream: Any) -> None:
        source = self._buffers[int(src.handle)]
        dst.view[: len(source)] = source

    def record_event(self, stream: Any) -> Any:
        return object()

    def destroy_event(self, event: Any) -> None:
        return None

    def wait_event(self, stream: Any, event: Any) -> None:
        return None

    def synchronize_stream(self, stream: Any) -> None:
        return None
