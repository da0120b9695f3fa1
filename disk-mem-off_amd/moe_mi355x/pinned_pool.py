"""Pinned host staging memory, lent out in exact byte sizes and fenced by copy events.

Interface of offload_runtime/pinned_pool.py:9-30 (``acquire(nbytes)``, ``release(buf)``,
``drain()``).  The design is this package's own: a staging buffer is handed back with the
event of the host->device copy that still reads it (``copy_event``), and the pool takes
ownership of that event.  The host waits on it only when the buffer is lent out again (the
caller is about to overwrite it), so ``release`` never blocks the loop that issues copies.
Buffers of one size are lent oldest-release first, the one whose copy most likely ended.
``max_idle_bytes`` bounds the pinned memory kept idle; beyond it a released buffer is freed
at once (after its copy).
"""
from __future__ import annotations

from collections import deque
from typing import Any, NamedTuple

from .backends import DeviceBackend
from .types import HostBuffer


class _Parked(NamedTuple):
    buf: HostBuffer
    fence: Any  # event of the last copy that reads ``buf`` (owned by the pool), or None


class PinnedHostBufferPool:
    """Lends pinned host buffers by exact size; each idle buffer carries the event of the
    copy that last read it, and the pool waits on that event before lending it again."""

    def __init__(self, backend: DeviceBackend, max_idle_bytes: int | None = None) -> None:
        self._backend = backend
        self._idle: dict[int, deque[_Parked]] = {}
        self.max_idle_bytes = max_idle_bytes
        self.idle_bytes = 0
        self.hits = 0    # acquisitions served from idle buffers
        self.misses = 0  # acquisitions that allocated

    @property
    def _free(self) -> dict[int, deque[_Parked]]:
        """Idle buffers by size (the attribute the reference's pool tests inspect)."""
        return self._idle

    def acquire(self, nbytes: int) -> HostBuffer:
        parked_of_size = self._idle.get(nbytes)
        if not parked_of_size:
            self.misses += 1
            return self._backend.alloc_pinned_host(nbytes)
        parked = parked_of_size.popleft()
        if not parked_of_size:
            del self._idle[nbytes]
        self.idle_bytes -= nbytes
        self.hits += 1
        self._settle(parked.fence)
        return parked.buf

    def release(self, buf: HostBuffer, copy_event: Any = None) -> None:
        """Return ``buf``; ``copy_event`` (owned by the pool from here on) marks the end of
        the last copy that reads it."""
        if not buf.pinned:
            raise ValueError("PinnedHostBufferPool.release: buffer is not pinned host memory")
        if self.max_idle_bytes is not None and self.idle_bytes + buf.nbytes > self.max_idle_bytes:
            self._settle(copy_event)
            self._backend.free_pinned_host(buf)
            return
        self._idle.setdefault(buf.nbytes, deque()).append(_Parked(buf, copy_event))
        self.idle_bytes += buf.nbytes

    def drain(self) -> None:
        """Free every idle buffer, each after the copy that reads it."""
        idle, self._idle = self._idle, {}
        self.idle_bytes = 0
        for parked_of_size in idle.values():
            for parked in parked_of_size:
                self._settle(parked.fence)
                self._backend.free_pinned_host(parked.buf)

    def _settle(self, fence: Any) -> None:
        if fence is None:
            return
        wait = getattr(self._backend, "event_synchronize", None)
        if wait is not None:
            wait(fence)
        self._backend.destroy_event(fence)
