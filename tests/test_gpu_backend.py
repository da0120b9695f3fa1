"""The ROCm backend through the C ABI (mirrors the reference's
tests/test_rocm_backend.py:28-85), plus the device data generators."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from moe_mi355x import _lib, gen
from moe_mi355x.moe import read_device
from moe_mi355x.quantize import quantize_rows_int8
from moe_mi355x.types import DeviceBuffer, HostBuffer

pytestmark = pytest.mark.gpu


def test_name_and_flags(mi355x):
    assert mi355x.name == "rocm"
    assert mi355x.supports_pinned_host is True
    assert mi355x.supports_peer_to_peer is True
    assert mi355x.supports_graph_capture is True


def test_stream_create_destroy(mi355x):
    s = mi355x.create_stream("test")
    assert s
    mi355x.destroy_stream(s)


def test_alloc_free_device(mi355x):
    buf = mi355x.alloc_device(64)
    assert isinstance(buf, DeviceBuffer) and buf.nbytes == 64 and buf.backend == "rocm"
    mi355x.free_device(buf)


def test_pinned_alloc_free(mi355x):
    buf = mi355x.alloc_pinned_host(64)
    assert buf.pinned is True and buf.nbytes == 64
    mi355x.free_pinned_host(buf)


def test_h2d_d2h_roundtrip(mi355x):
    data = bytearray(b"rocm test data!!")
    src = HostBuffer(view=memoryview(bytearray(data)), pinned=False)
    dev = mi355x.alloc_device(16)
    s = mi355x.create_stream("xfer")
    try:
        mi355x.copy_h2d_async(dev, src, s)
        dst = HostBuffer(view=memoryview(bytearray(16)), pinned=False)
        mi355x.copy_d2h_async(dst, dev, s)
        mi355x.synchronize_stream(s)
        assert bytes(dst.view) == bytes(data)
    finally:
        mi355x.free_device(dev)
        mi355x.destroy_stream(s)


def test_copy_size_and_readonly_errors(mi355x):
    dev = mi355x.alloc_device(32)
    s = mi355x.create_stream("x")
    try:
        with pytest.raises(ValueError):
            mi355x.copy_h2d_async(dev, HostBuffer(memoryview(bytearray(16))), s)
        with pytest.raises(ValueError):
            mi355x.copy_d2h_async(HostBuffer(memoryview(bytearray(16))), dev, s)
        with pytest.raises(ValueError):
            mi355x.copy_h2d_async(dev, HostBuffer(memoryview(bytes(32))), s)
    finally:
        mi355x.free_device(dev)
        mi355x.destroy_stream(s)


def test_event_record_wait(mi355x):
    s1, s2 = mi355x.create_stream("s1"), mi355x.create_stream("s2")
    ev = mi355x.record_event(s1)
    mi355x.wait_event(s2, ev)
    mi355x.synchronize_stream(s2)
    assert mi355x.event_done(ev)
    mi355x.destroy_event(ev)
    mi355x.destroy_stream(s1)
    mi355x.destroy_stream(s2)


def test_hip_error_becomes_runtime_error(mi355x):
    with pytest.raises(RuntimeError, match="status="):
        _lib.check(_lib.load().mx_set_device(1 << 20), "hipSetDevice")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_fill_normal_matches_host_generator(mi355x, stream, dtype):
    n, off = 1 << 20, 12345
    code = _lib.MX_DT_F32 if dtype == "float32" else _lib.MX_DT_F16
    dev = mi355x.alloc_device(n * 4)
    try:
        _lib.check(_lib.load().mx_fill_normal(dev.handle, code, n, 99, 7, off, 0.02, stream))
        got = read_device(mi355x, dev.handle, np.dtype(dtype), n, stream)
    finally:
        mi355x.free_device(dev)
    want = gen.normal(99, 7, (n,), std=0.02, offset=off, dtype=np.dtype(dtype))
    same = got == want
    # log/cos of two libms may differ in the last fp64 ulp; that flips a rounding of the
    # stored value only in rare elements, and never by more than one ulp.
    assert same.mean() > 0.9999
    if not same.all():
        gi = got[~same].astype(np.float64)
        wi = want[~same].astype(np.float64)
        assert np.all(np.abs(gi - wi) <= np.spacing(np.abs(wi).astype(dtype)).astype(np.float64))


def test_quantize_rows_device_matches_host(mi355x, stream):
    rows, cols = 96, 320
    w = gen.normal(5, 1, (rows, cols), std=0.02)
    w[3] = 0.0
    dev = mi355x.alloc_device(w.nbytes + rows * cols + rows * 2 + 256)
    try:
        q_off = w.nbytes
        s_off = q_off + rows * cols
        pin = np.ascontiguousarray(w)
        mi355x.copy_h2d_ptr_async(dev.handle, pin.ctypes.data, w.nbytes, stream)
        mi355x.synchronize_stream(stream)
        _lib.check(_lib.load().mx_quantize_rows_i8(dev.handle, _lib.MX_DT_F32, rows, cols,
                                                   dev.handle + q_off, dev.handle + s_off, stream))
        q = read_device(mi355x, dev.handle + q_off, np.int8, rows * cols, stream).reshape(rows, cols)
        s = read_device(mi355x, dev.handle + s_off, np.float16, rows, stream)
    finally:
        mi355x.free_device(dev)
    q2, s2 = quantize_rows_int8(w)
    assert np.array_equal(s.view(np.uint16), s2.view(np.uint16))
    assert np.array_equal(q, q2)
