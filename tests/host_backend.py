"""A CPU fake of a device backend for the CPU tests of the runtime, the pools and the
executors' host logic.

Design: "device memory" is a set of NumPy byte arrays keyed by fake, 256-byte aligned
device addresses handed out by a bump counter (so handles look like device addresses and
never collide with host ids); every stream keeps a log of the operations enqueued on it;
events count themselves so a test can check that a run leaked none.  Copies complete at
once.  The MoE step itself never runs here: the product package has no CPU path, and an
executor handed this backend raises.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np

from moe_mi355x.backends import DeviceBackend
from moe_mi355x.types import DeviceBuffer, HostBuffer

_ALIGN = 256
_BASE = 0x7F00_0000_0000


@dataclass
class FakeStream:
    purpose: str
    log: list = field(default_factory=list)  # ("h2d" | "d2h" | "wait" | "record", n)


@dataclass
class FakeEvent:
    serial: int
    stream: FakeStream | None


class HostArenaBackend(DeviceBackend):
    """Device buffers are NumPy byte arrays at fake device addresses; copies are
    synchronous; streams log their operations; events are counted."""

    name = "host-arena"

    def __init__(self) -> None:
        self.allocations: dict[int, np.ndarray] = {}
        self.pinned: dict[int, np.ndarray] = {}
        self.live_events = 0
        self._next_address = _BASE
        self._serial = 0

    # -- memory --
    @property
    def supports_pinned_host(self) -> bool:
        return True

    def alloc_device(self, nbytes: int) -> DeviceBuffer:
        address = self._next_address
        self._next_address += (max(nbytes, 1) + _ALIGN - 1) // _ALIGN * _ALIGN
        self.allocations[address] = np.zeros(nbytes, np.uint8)
        return DeviceBuffer(handle=address, nbytes=nbytes, backend=self.name)

    def free_device(self, buf: DeviceBuffer) -> None:
        if self.allocations.pop(int(buf.handle), None) is None:
            raise ValueError(f"free of unknown device address {int(buf.handle):#x}")

    def alloc_pinned_host(self, nbytes: int) -> HostBuffer:
        arr = np.zeros(nbytes, np.uint8)
        self.pinned[id(arr)] = arr
        return HostBuffer(view=memoryview(arr), pinned=True)

    def free_pinned_host(self, buf: HostBuffer) -> None:
        self.pinned.pop(id(buf.view.obj), None)

    def device_bytes(self, buf: DeviceBuffer) -> bytes:
        return self.allocations[int(buf.handle)].tobytes()

    # -- streams, copies, events --
    def create_stream(self, purpose: str) -> FakeStream:
        return FakeStream(purpose)

    def destroy_stream(self, stream: Any) -> None:
        return None

    def copy_h2d_async(self, dst: DeviceBuffer, src: HostBuffer, stream: Any) -> None:
        data = np.frombuffer(src.view, np.uint8)
        target = self.allocations[int(dst.handle)]
        if data.size > target.size:
            raise ValueError("source is larger than the device buffer")
        target[: data.size] = data
        if isinstance(stream, FakeStream):
            stream.log.append(("h2d", int(data.size)))

    def copy_d2h_async(self, dst: HostBuffer, src: DeviceBuffer, stream: Any) -> None:
        source = self.allocations[int(src.handle)]
        out = np.frombuffer(dst.view, np.uint8)
        if out.size < source.size:
            raise ValueError("destination is smaller than the device buffer")
        out[: source.size] = source
        if isinstance(stream, FakeStream):
            stream.log.append(("d2h", int(source.size)))

    def record_event(self, stream: Any) -> FakeEvent:
        self._serial += 1
        self.live_events += 1
        if isinstance(stream, FakeStream):
            stream.log.append(("record", self._serial))
        return FakeEvent(self._serial, stream if isinstance(stream, FakeStream) else None)

    def destroy_event(self, event: Any) -> None:
        if event is not None:
            self.live_events -= 1

    def wait_event(self, stream: Any, event: Any) -> None:
        if isinstance(stream, FakeStream) and isinstance(event, FakeEvent):
            stream.log.append(("wait", event.serial))

    def event_synchronize(self, event: Any) -> None:
        return None

    def event_done(self, event: Any) -> bool:
        return True

    def synchronize_stream(self, stream: Any) -> None:
        return None
