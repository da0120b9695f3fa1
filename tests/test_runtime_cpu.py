"""OffloadRuntime on the CPU backend: the reference's runtime contract
(tests/test_runtime.py:14-386 of the reference) plus the transfer-ahead schedule."""
from __future__ import annotations

import struct
from typing import Any

import pytest

from host_backend import HostArenaBackend
from moe_mi355x.quantize import CompositeDequantizer, Int8Dequantizer
from moe_mi355x.runtime import OffloadRuntime, RuntimeMetrics
from moe_mi355x.scheduler import LookaheadScheduler
from moe_mi355x.storage import InMemoryStorage
from moe_mi355x.types import DeviceBuffer, LayerSpec


class SumExecutor:
    def run_layer(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                  backend: Any, stream: Any) -> int:
        return activations + layer.layer_id


class RecordingExecutor:
    """Records the order of layers and the bytes it saw on the device."""

    def __init__(self) -> None:
        self.executed: list[int] = []
        self.payloads: list[bytes] = []

    def run_layer(self, layer, activations, device_weights, backend, stream):
        self.executed.append(layer.layer_id)
        self.payloads.append(backend.device_bytes(device_weights))
        return activations


def layers(n: int, nbytes: int = 16) -> list[LayerSpec]:
    return [LayerSpec(layer_id=i, name=f"L{i}", nbytes=nbytes) for i in range(n)]


def storage(n: int, nbytes: int = 16) -> InMemoryStorage:
    return InMemoryStorage({i: bytes([i]) * nbytes for i in range(n)})


def runtime(n=3, lookahead=1, **kw) -> OffloadRuntime:
    backend = kw.pop("backend", HostArenaBackend())
    return OffloadRuntime(layers=layers(n), backend=backend, storage=storage(n),
                          scheduler=LookaheadScheduler(lookahead=lookahead),
                          executor=kw.pop("executor", SumExecutor()), **kw)


@pytest.mark.parametrize("lookahead", [0, 1, 2, 5])
def test_sum_and_order(lookahead):
    ex = RecordingExecutor()
    rt = runtime(5, lookahead, executor=ex)
    out, m = rt.run_inference([0, 1, 2, 3, 4], inputs=0)
    assert ex.executed == [0, 1, 2, 3, 4]
    # every layer saw its own bytes even with several copies in flight
    assert ex.payloads == [bytes([i]) * 16 for i in range(5)]
    assert m.layer_count == 5


def test_sum_executor():
    out, _ = runtime(5, 2).run_inference([0, 1, 2, 3, 4], inputs=0)
    assert out == 10


def test_unknown_layer_raises():
    with pytest.raises(ValueError, match="Unknown layer IDs"):
        runtime(2).run_inference([0, 7], inputs=0)


def test_device_buffers_freed():
    backend = HostArenaBackend()
    runtime(3, 2, backend=backend).run_inference([0, 1, 2], inputs=0)
    assert len(backend.allocations) == 0


def test_per_layer_metrics():
    _, m = runtime(3, 1).run_inference([0, 1, 2], inputs=0)
    assert [lm.layer_id for lm in m.layer_metrics] == [0, 1, 2]
    for lm in m.layer_metrics:
        assert lm.nbytes == 16 and lm.h2d_ms >= 0 and lm.compute_ms >= 0 and lm.stall_ms >= 0
    assert m.end_to_end_seconds > 0 and m.transferred_bytes == 48


def test_metric_formulas():
    assert RuntimeMetrics(transferred_bytes=10 ** 9, transfer_seconds=1.0).effective_bandwidth_gbps \
        == pytest.approx(1.0)
    assert RuntimeMetrics(transferred_bytes=100).effective_bandwidth_gbps == 0.0
    assert RuntimeMetrics(transfer_seconds=1, compute_seconds=1,
                          end_to_end_seconds=2).overlap_ratio == pytest.approx(0.0)
    assert RuntimeMetrics(transfer_seconds=1, compute_seconds=1,
                          end_to_end_seconds=1).overlap_ratio == pytest.approx(0.5)
    assert RuntimeMetrics(transfer_gpu_seconds=1, compute_gpu_seconds=1,
                          device_seconds=1).gpu_overlap_ratio == pytest.approx(0.5)


def test_buffer_pool_and_pinned_staging():
    backend = HostArenaBackend()
    with runtime(3, 2, backend=backend, use_buffer_pool=True, use_pinned_staging=True) as rt:
        out, m = rt.run_inference([0, 1, 2], inputs=0)
        assert out == 3 and m.transferred_bytes == 48
    # every device buffer, pinned staging buffer and event is released at close
    assert len(backend.allocations) == 0 and len(backend.pinned) == 0
    assert backend.live_events == 0


def test_pinned_staging_skipped_when_unsupported():
    class NoPinned(HostArenaBackend):
        @property
        def supports_pinned_host(self) -> bool:
            return False

    with runtime(2, 1, backend=NoPinned(), use_pinned_staging=True) as rt:
        assert rt.run_inference([0, 1], inputs=0)[0] == 1


def test_quantized_transfer_accounting():
    lay = [LayerSpec(0, "L0", 4, {"dtype": "int8", "scale": 1.0}),
           LayerSpec(1, "L1", 4, {"dtype": "int8", "scale": 1.0})]
    st = InMemoryStorage({0: struct.pack("4b", 1, 2, 3, 4), 1: struct.pack("4b", 5, 6, 7, 8)})
    rt = OffloadRuntime(lay, HostArenaBackend(), st, LookaheadScheduler(1), SumExecutor(),
                        dequantizer=Int8Dequantizer())
    out, m = rt.run_inference([0, 1], inputs=0)
    assert out == 1 and m.transferred_bytes == 32 and m.compressed_bytes == 8
    assert m.layer_metrics[0].compressed_nbytes == 4 and m.layer_metrics[0].nbytes == 16


def test_quantized_mixed_layers():
    lay = [LayerSpec(0, "L0", 16), LayerSpec(1, "L1", 4, {"dtype": "int8", "scale": 1.0})]
    st = InMemoryStorage({0: b"\x00" * 16, 1: struct.pack("4b", 1, 2, 3, 4)})
    rt = OffloadRuntime(lay, HostArenaBackend(), st, LookaheadScheduler(1), SumExecutor(),
                        dequantizer=CompositeDequantizer())
    _, m = rt.run_inference([0, 1], inputs=0)
    assert m.transferred_bytes == 32 and m.compressed_bytes == 4
    assert [lm.compressed_nbytes for lm in m.layer_metrics] == [0, 4]


def test_transfer_lookahead_defaults_to_scheduler_window():
    assert runtime(2, 2).transfer_lookahead == 2
    assert runtime(2, 0).transfer_lookahead == 0
    with pytest.raises(ValueError):
        runtime(2, 1, transfer_lookahead=-1)


def test_transfers_issued_ahead_of_compute():
    """With a window of 2, the copies of layers i+1 and i+2 are enqueued before layer i
    runs (the reference enqueues copy i right before compute i)."""
    events: list[str] = []

    class Spy(HostArenaBackend):
        def copy_h2d_async(self, dst, src, stream):
            events.append(f"copy{src.view.tobytes()[0]}")
            super().copy_h2d_async(dst, src, stream)

    class Ex:
        def run_layer(self, layer, activations, device_weights, backend, stream):
            events.append(f"run{layer.layer_id}")
            return activations

    rt = runtime(4, 2, backend=Spy(), executor=Ex())
    rt.run_inference([0, 1, 2, 3], inputs=0)
    assert events == ["copy0", "copy1", "copy2", "run0", "copy3", "run1", "run2", "run3"]


def test_expert_granular_needs_capable_executor_and_backend():
    from host_backend import HostArenaBackend
    from moe_mi355x.runtime import OffloadRuntime
    from moe_mi355x.scheduler import LookaheadScheduler
    from moe_mi355x.storage import InMemoryStorage

    class Plain:
        def run_layer(self, layer, activations, device_weights, backend, stream):
            return activations

    class Granular(Plain):
        def run_layer_granular(self, layer, activations, device_weights, backend, stream, fetch):
            return activations

        def expert_ranges(self, layer):
            return [], []

    with pytest.raises(ValueError, match="run_layer_granular"):
        OffloadRuntime([], HostArenaBackend(), InMemoryStorage({}), LookaheadScheduler(1), Plain(),
                       expert_granular=True)
    with pytest.raises(ValueError, match="pointer copies"):
        OffloadRuntime([], HostArenaBackend(), InMemoryStorage({}), LookaheadScheduler(1), Granular(),
                       expert_granular=True)


def test_resident_layers_are_neither_copied_nor_freed():
    from moe_mi355x.storage import DeviceResidentStorage

    backend = HostArenaBackend()
    bufs = {i: backend.alloc_device(16) for i in range(3)}
    seen = []

    class Ex:
        stream_ordered = False

        def run_layer(self, layer, activations, device_weights, backend, stream):
            seen.append(device_weights.handle)
            return activations + 1

    ex = Ex()
    rt = OffloadRuntime(layers(3), backend, DeviceResidentStorage(bufs), LookaheadScheduler(2),
                        ex, use_buffer_pool=True)
    with rt:
        out, m = rt.run_inference([0, 1, 2, 1], inputs=0)
    assert out == 4 and m.transferred_bytes == 0 and ex.stream_ordered
    assert seen == [bufs[i].handle for i in (0, 1, 2, 1)]
    assert len(backend.allocations) == 3 and backend.live_events == 0
    assert not any(op[0] == "h2d" for op in rt.transfer_stream.log)


def test_device_activations_come_back_as_numpy():
    """An executor that keeps activations on the device: the runtime returns NumPy when
    it was given NumPy (the reference contract); a stale handle refuses to read."""
    import ctypes

    import numpy as np

    from moe_mi355x.activations import DeviceActivations

    class Owner:
        def __init__(self):
            self.gen = [0, 0, 0]
            self.backend = self

        def generation(self, slot):
            return self.gen[slot]

        def copy_d2h_ptr_async(self, dst, src, nbytes, stream):
            ctypes.memmove(dst, src, nbytes)

        def synchronize_stream(self, stream):
            return None

    owner = Owner()
    store = [np.zeros((2, 4), np.float32) for _ in range(3)]

    class Ex:
        stream_ordered = False

        def __init__(self):
            self.k = 0

        def run_layer(self, layer, activations, device_weights, backend, stream):
            x = np.asarray(activations, np.float32)
            slot = 1 + self.k % 2
            self.k += 1
            store[slot][:] = x + 1
            owner.gen[slot] += 1
            return DeviceActivations(owner, slot, owner.gen[slot], store[slot].ctypes.data,
                                     2, 4, None)

    rt = OffloadRuntime(layers(2), HostArenaBackend(), storage(2), LookaheadScheduler(1), Ex())
    with rt:
        out, _ = rt.run_inference([0, 1, 0], np.zeros((2, 4), np.float32))
    assert isinstance(out, np.ndarray) and np.all(out == 3)
    h = DeviceActivations(owner, 1, owner.gen[1], store[1].ctypes.data, 2, 4, None)
    owner.gen[1] += 1
    with pytest.raises(RuntimeError, match="overwritten"):
        h.numpy()
