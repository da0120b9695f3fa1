"""Exact-size free list for pinned host buffers (offload_runtime/pinned_pool.py:9-30):
``acquire(n)`` pops a released buffer of exactly ``n`` bytes or allocates one with
``alloc_pinned_host``; ``release`` returns it to its size class; ``drain`` frees all.

Host staging buffers are reused only after the runtime has waited for the copy that read
them (the runtime holds a staged buffer until its layer's H2D event completed), so no
event travels with them here, unlike the device pool.
"""
from __future__ import annotations

from collections import defaultdict

from .backends import DeviceBackend
from .types import HostBuffer


class PinnedHostBufferPool:
    """Reuses pinned host buffers of the same size to avoid frequent alloc/free."""

    def __init__(self, backend: DeviceBackend) -> None:
        self._backend = backend
        self._free: dict[int, list[HostBuffer]] = defaultdict(list)

    def acquire(self, nbytes: int) -> HostBuffer:
        pool = self._free.get(nbytes)
        if pool:
            return pool.pop()
        return self._backend.alloc_pinned_host(nbytes)

    def release(self, buf: HostBuffer) -> None:
        self._free[buf.nbytes].append(buf)

    def drain(self) -> None:
        for pool in self._free.values():
            for buf in pool:
                self._backend.free_pinned_host(buf)
            pool.clear()
        self._free.clear()
