"""Exact-size free list for device buffers.

Behaviour of offload_runtime/buffer_pool.py:9-30:
``acquire(n)`` pops a released buffer of exactly ``n`` bytes or allocates a new one,
``release`` returns a buffer to its size class, ``drain`` frees everything.

Device reuse on a GPU is asynchronous: a buffer released while kernels still read it may
be handed to the next copy.  ``release(buf, ready_event=ev)`` records the event after
which the buffer is free; ``acquire`` hands it back together with that event
(``last_event``) so the caller can make its stream wait before overwriting it.
"""
from __future__ import annotations

from collections import defaultdict
from typing import Any

from .backends import DeviceBackend
from .types import DeviceBuffer


class DeviceBufferPool:
    """Reuses device buffers of the same size to avoid frequent malloc/free."""

    def __init__(self, backend: DeviceBackend) -> None:
        self._backend = backend
        self._free: dict[int, list[tuple[DeviceBuffer, Any]]] = defaultdict(list)
        self.last_event: Any = None

    def acquire(self, nbytes: int) -> DeviceBuffer:
        pool = self._free.get(nbytes)
        if pool:
            buf, ev = pool.pop()
            self.last_event = ev
            return buf
        self.last_event = None
        return self._backend.alloc_device(nbytes)

    def release(self, buf: DeviceBuffer, ready_event: Any = None) -> None:
        self._free[buf.nbytes].append((buf, ready_event))

    def drain(self) -> None:
        for pool in self._free.values():
            for buf, ev in pool:
                if ev is not None:
                    self._backend.destroy_event(ev)
                self._backend.free_device(buf)
            pool.clear()
        self._free.clear()
