"""Device / pinned buffer pools on the CPU fake backend (the cases of the reference's
tests/test_buffer_pool.py:12-50 and tests/test_pinned_pool.py:12-48, plus the event fences
of this package's pools)."""
from __future__ import annotations

import pytest

from host_backend import HostArenaBackend
from moe_mi355x.buffer_pool import DeviceBufferPool
from moe_mi355x.pinned_pool import PinnedHostBufferPool


class TestDeviceBufferPool:
    def setup_method(self):
        self.backend = HostArenaBackend()
        self.pool = DeviceBufferPool(self.backend)

    def test_acquire_allocates_new(self):
        buf = self.pool.acquire(64)
        assert buf.nbytes == 64 and buf.backend == "host-arena"

    def test_release_and_reuse(self):
        b1 = self.pool.acquire(64)
        self.pool.release(b1)
        assert self.pool.acquire(64).handle == b1.handle

    def test_different_sizes_not_reused(self):
        b1 = self.pool.acquire(32)
        self.pool.release(b1)
        assert self.pool.acquire(64).handle != b1.handle

    def test_drain_frees_all(self):
        b1, b2 = self.pool.acquire(32), self.pool.acquire(32)
        self.pool.release(b1)
        self.pool.release(b2)
        assert len(self.backend.allocations) == 2
        self.pool.drain()
        assert len(self.backend.allocations) == 0

    def test_cycles_reuse_one_buffer(self):
        handles = set()
        for _ in range(5):
            b = self.pool.acquire(16)
            handles.add(b.handle)
            self.pool.release(b)
        assert len(handles) == 1

    def test_ready_event_is_handed_back(self):
        b = self.pool.acquire(16)
        ev = object()
        self.pool.release(b, ready_event=ev)
        assert self.pool.acquire(16).handle == b.handle and self.pool.last_event is ev
        self.pool.acquire(16)
        assert self.pool.last_event is None


class TestPinnedHostBufferPool:
    def setup_method(self):
        self.backend = HostArenaBackend()
        self.pool = PinnedHostBufferPool(self.backend)

    def test_acquire_allocates_pinned(self):
        buf = self.pool.acquire(64)
        assert buf.pinned is True and buf.nbytes == 64

    def test_release_and_reuse(self):
        b1 = self.pool.acquire(64)
        obj = b1.view.obj
        self.pool.release(b1)
        assert self.pool.acquire(64).view.obj is obj

    def test_different_sizes_not_reused(self):
        b1 = self.pool.acquire(32)
        self.pool.release(b1)
        b2 = self.pool.acquire(64)
        assert b2.nbytes == 64 and b2.view.obj is not b1.view.obj

    def test_drain(self):
        b1, b2 = self.pool.acquire(32), self.pool.acquire(32)
        self.pool.release(b1)
        self.pool.release(b2)
        self.pool.drain()
        assert len(self.pool._free) == 0

    def test_multiple_cycles(self):
        objs = set()
        for _ in range(5):
            b = self.pool.acquire(16)
            objs.add(id(b.view.obj))
            self.pool.release(b)
        assert len(objs) == 1 and self.pool.hits == 4 and self.pool.misses == 1

    def test_copy_event_is_waited_on_before_reuse(self):
        waited = []
        self.backend.event_synchronize = waited.append
        b = self.pool.acquire(64)
        ev = self.backend.record_event(None)
        self.pool.release(b, copy_event=ev)
        assert waited == [] and self.backend.live_events == 1  # release does not block
        assert self.pool.acquire(64).view.obj is b.view.obj
        assert waited == [ev] and self.backend.live_events == 0  # waited, then destroyed

    def test_drain_settles_events_and_frees(self):
        b1, b2 = self.pool.acquire(8), self.pool.acquire(8)
        self.pool.release(b1, copy_event=self.backend.record_event(None))
        self.pool.release(b2)
        assert self.pool.idle_bytes == 16
        self.pool.drain()
        assert self.backend.live_events == 0 and len(self.backend.pinned) == 0
        assert self.pool.idle_bytes == 0

    def test_oldest_release_is_lent_first(self):
        b1, b2 = self.pool.acquire(8), self.pool.acquire(8)
        self.pool.release(b1)
        self.pool.release(b2)
        assert self.pool.acquire(8).view.obj is b1.view.obj

    def test_idle_cap_frees_beyond_it(self):
        pool = PinnedHostBufferPool(self.backend, max_idle_bytes=16)
        bufs = [pool.acquire(8) for _ in range(3)]
        for b in bufs:
            pool.release(b)
        assert pool.idle_bytes == 16 and len(self.backend.pinned) == 2

    def test_unpinned_release_rejected(self):
        from moe_mi355x.types import HostBuffer
        with pytest.raises(ValueError, match="not pinned"):
            self.pool.release(HostBuffer(view=memoryview(bytearray(8))))
