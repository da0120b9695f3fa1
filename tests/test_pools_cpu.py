"""Device / pinned buffer pools on the CPU backend (mirrors the reference's
tests/test_buffer_pool.py:12-50 and tests/test_pinned_pool.py:12-48)."""
from __future__ import annotations

from null_backend import NullBackend
from moe_mi355x.buffer_pool import DeviceBufferPool
from moe_mi355x.pinned_pool import PinnedHostBufferPool


class TestDeviceBufferPool:
    def setup_method(self):
        self.backend = NullBackend()
        self.pool = DeviceBufferPool(self.backend)

    def test_acquire_allocates_new(self):
        buf = self.pool.acquire(64)
        assert buf.nbytes == 64 and buf.backend == "null"

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
        assert len(self.backend._buffers) == 2
        self.pool.drain()
        assert len(self.backend._buffers) == 0

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
        self.backend = NullBackend()
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
