"""Device memory for layer weights, lent out in exact byte sizes and fenced by events.

Interface of offload_runtime/buffer_pool.py:9-30 (``acquire(nbytes)``, ``release(buf)``,
``drain()``).  On a GPU a buffer comes back while kernels may still read it, and the pool
may lend it straight to the next host->device copy.  So a buffer is returned with the event
after which it is free (``release(buf, ready_event=ev)``), and ``acquire`` exposes that
event as ``last_event``: the caller makes its copy stream wait on it (a device-side wait, no
host block) and then owns the event.  Buffers of one size are lent oldest-release first,
the one whose last reader most likely finished.
"""
from __future__ import annotations

from collections import deque
from typing import Any, NamedTuple

from .backends import DeviceBackend
from .types import DeviceBuffer


class _Parked(NamedTuple):
    buf: DeviceBuffer
    fence: Any  # event after which ``buf`` may be overwritten, or None


class DeviceBufferPool:
    """Lends device buffers by exact size; an idle buffer carries the event that ends its
    last use, handed to the next borrower as ``last_event``."""

    def __init__(self, backend: DeviceBackend) -> None:
        self._backend = backend
        self._idle: dict[int, deque[_Parked]] = {}
        self.last_event: Any = None
        self.hits = 0
        self.misses = 0

    @property
    def _free(self) -> dict[int, deque[_Parked]]:
        """Idle buffers by size (the attribute the reference's pool tests inspect)."""
        return self._idle

    def acquire(self, nbytes: int) -> DeviceBuffer:
        parked_of_size = self._idle.get(nbytes)
        if not parked_of_size:
            self.misses += 1
            self.last_event = None
            return self._backend.alloc_device(nbytes)
        parked = parked_of_size.popleft()
        if not parked_of_size:
            del self._idle[nbytes]
        self.hits += 1
        self.last_event = parked.fence
        return parked.buf

    def release(self, buf: DeviceBuffer, ready_event: Any = None) -> None:
        self._idle.setdefault(buf.nbytes, deque()).append(_Parked(buf, ready_event))

    def drain(self) -> None:
        """Free every idle buffer (the caller has synchronised the streams that used them)."""
        idle, self._idle = self._idle, {}
        for parked_of_size in idle.values():
            for parked in parked_of_size:
                if parked.fence is not None:
                    self._backend.destroy_event(parked.fence)
                self._backend.free_device(parked.buf)
