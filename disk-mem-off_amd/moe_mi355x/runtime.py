"""Layer-offload runtime with host->device transfers issued ahead of compute.

API and metrics of offload_runtime/runtime.py:15-198 (``LayerExecutor``, ``LayerMetrics``,
``RuntimeMetrics``, ``OffloadRuntime.run_inference``): storage wait -> optional host
dequantisation -> pinned staging -> device buffer (pool) -> H2D on the transfer stream ->
event -> ``run_layer`` on the compute stream -> release -> next storage prefetch.

Difference in scheduling: the reference enqueues the copy of layer i immediately before
computing layer i, so copies never overlap compute.  Here the copies of layers
i+1 .. i+transfer_lookahead are enqueued on the transfer stream *before* layer i runs on
the compute stream (``transfer_lookahead`` defaults to the scheduler's ``lookahead``;
0 restores the reference order).  Buffer hazards are fenced with events: a device buffer
goes back to the pool together with the event that marks the end of its compute, and the
next copy into it waits on that event on the transfer stream; a pinned staging buffer is
reused only after the event of its copy has completed.
"""
from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field
from typing import Any, Protocol

from .backends import DeviceBackend
from .activations import DeviceActivations
from .buffer_pool import DeviceBufferPool
from .pinned_pool import PinnedHostBufferPool
from .scheduler import PrefetchScheduler
from .storage import LayerStorage
from .types import DeviceBuffer, HostBuffer, LayerSpec


class LayerExecutor(Protocol):
    """Executes one layer using device weights already copied to the device."""

    def run_layer(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                  backend: DeviceBackend, stream: Any) -> Any: ...


@dataclass
class LayerMetrics:
    layer_id: int
    h2d_ms: float = 0.0          # host time to enqueue the copy (reference meaning)
    compute_ms: float = 0.0      # host wall time of run_layer
    stall_ms: float = 0.0
    disk_read_ms: float = 0.0
    nbytes: int = 0
    compressed_nbytes: int = 0
    h2d_gpu_ms: float = 0.0      # event-timed copy on the transfer stream (GPU backends)
    compute_gpu_ms: float = 0.0  # event-timed run_layer work on the compute stream


@dataclass
class RuntimeMetrics:
    transferred_bytes: int = 0
    compressed_bytes: int = 0
    transfer_seconds: float = 0.0
    compute_seconds: float = 0.0
    layer_count: int = 0
    end_to_end_seconds: float = 0.0
    layer_metrics: list[LayerMetrics] = field(default_factory=list)
    transfer_gpu_seconds: float = 0.0
    compute_gpu_seconds: float = 0.0
    device_seconds: float = 0.0  # event-timed first copy start -> last compute end

    @property
    def effective_bandwidth_gbps(self) -> float:
        if self.transfer_seconds <= 0:
            return 0.0
        return (self.transferred_bytes / 1e9) / self.transfer_seconds

    @property
    def overlap_ratio(self) -> float:
        """1 - e2e / (transfer + compute), the reference formula (runtime.py:56-61)."""
        total = self.transfer_seconds + self.compute_seconds
        if total <= 0 or self.end_to_end_seconds <= 0:
            return 0.0
        return 1.0 - (self.end_to_end_seconds / total)

    @property
    def gpu_transfer_bandwidth_gbps(self) -> float:
        if self.transfer_gpu_seconds <= 0:
            return 0.0
        return (self.transferred_bytes / 1e9) / self.transfer_gpu_seconds

    @property
    def gpu_overlap_ratio(self) -> float:
        """Same formula on event-timed device intervals."""
        total = self.transfer_gpu_seconds + self.compute_gpu_seconds
        if total <= 0 or self.device_seconds <= 0:
            return 0.0
        return 1.0 - (self.device_seconds / total)


@dataclass
class _Inflight:
    index: int
    layer: LayerSpec
    lm: LayerMetrics
    host: HostBuffer
    staged: HostBuffer
    device: DeviceBuffer
    copied: Any  # event recorded after the copy on the transfer stream
    t_start: Any = None  # timing events (GPU backends)
    t_end: Any = None
    granular: bool = False  # routed experts are copied on demand
    extra_copies: list = field(default_factory=list)  # timing events of on-demand copies
    resident: bool = False  # the storage handed over a device buffer it keeps


class OffloadRuntime:
    def __init__(
        self,
        layers: list[LayerSpec],
        backend: DeviceBackend,
        storage: LayerStorage,
        scheduler: PrefetchScheduler,
        executor: LayerExecutor,
        use_buffer_pool: bool = False,
        use_pinned_staging: bool = False,
        dequantizer: Any | None = None,
        transfer_lookahead: int | None = None,
        expert_granular: bool = False,
        event_timing: bool = True,
    ) -> None:
        self.layers = {layer.layer_id: layer for layer in layers}
        self.backend = backend
        self.storage = storage
        self.scheduler = scheduler
        self.executor = executor
        self.transfer_stream = backend.create_stream("transfer")
        self.compute_stream = backend.create_stream("compute")
        self._pool = DeviceBufferPool(backend) if use_buffer_pool else None
        self._pinned_pool: PinnedHostBufferPool | None = None
        if use_pinned_staging and backend.supports_pinned_host:
            self._pinned_pool = PinnedHostBufferPool(backend)
        self.dequantizer = dequantizer
        if transfer_lookahead is None:
            transfer_lookahead = int(getattr(scheduler, "lookahead", 0))
        if transfer_lookahead < 0:
            raise ValueError("transfer_lookahead must be >= 0")
        self.transfer_lookahead = transfer_lookahead
        self._timing = bool(event_timing) and hasattr(backend, "create_timing_event")
        # Every buffer this runtime frees or re-pools after run_layer is fenced by an event
        # recorded on the compute stream after the call, so an executor that can return
        # before its device work ends may do so.
        if hasattr(executor, "stream_ordered"):
            executor.stream_ordered = True
        self._deferred_free: list[tuple[DeviceBuffer, Any]] = []
        # Expert-granular transfer: ahead of compute only the bytes outside the routed
        # experts are copied; after the layer's router has run, the executor asks for the
        # routed experts it needs (run_layer_granular + fetch).
        self.expert_granular = bool(expert_granular)
        if self.expert_granular:
            if not hasattr(executor, "run_layer_granular"):
                raise ValueError("expert_granular needs an executor with run_layer_granular")
            if not hasattr(backend, "copy_h2d_ptr_async"):
                raise ValueError("expert_granular needs a backend with pointer copies")
            if dequantizer is not None:
                raise ValueError("expert_granular copies raw layer bytes; no host dequantizer")

    def __enter__(self) -> "OffloadRuntime":
        return self

    def __exit__(self, exc_type: Any, exc_val: Any, exc_tb: Any) -> None:
        self.close()

    def close(self) -> None:
        self.backend.synchronize_stream(self.transfer_stream)
        self.backend.synchronize_stream(self.compute_stream)
        self._flush_deferred(force=True)
        if self._pinned_pool is not None:
            self._pinned_pool.drain()
        if self._pool is not None:
            self._pool.drain()
        self.backend.destroy_stream(self.transfer_stream)
        self.backend.destroy_stream(self.compute_stream)

    # -- buffers --
    def _alloc_device(self, nbytes: int) -> DeviceBuffer:
        if self._pool is not None:
            buf = self._pool.acquire(nbytes)
            ev = self._pool.last_event
            if ev is not None:
                # The previous user of this buffer must finish before the copy lands.
                self.backend.wait_event(self.transfer_stream, ev)
                self.backend.destroy_event(ev)
            return buf
        return self.backend.alloc_device(nbytes)

    def _free_device(self, buf: DeviceBuffer, done_event: Any) -> None:
        if self._pool is not None:
            self._pool.release(buf, done_event)
        elif done_event is None:
            self.backend.free_device(buf)
        else:
            self._deferred_free.append((buf, done_event))

    def _flush_deferred(self, force: bool = False) -> None:
        keep = []
        for buf, ev in self._deferred_free:
            if force or self._event_done(ev):
                self.backend.destroy_event(ev)
                self.backend.free_device(buf)
            else:
                keep.append((buf, ev))
        self._deferred_free = keep

    def _event_done(self, ev: Any) -> bool:
        query = getattr(self.backend, "event_done", None)
        return True if query is None else bool(query(ev))

    def _stage_pinned(self, host_weights: HostBuffer) -> HostBuffer:
        if self._pinned_pool is None or host_weights.pinned:
            return host_weights
        pinned = self._pinned_pool.acquire(host_weights.nbytes)
        pinned.view[: host_weights.nbytes] = host_weights.view[: host_weights.nbytes]
        return pinned

    def _release_staging(self, rec: _Inflight) -> None:
        """Hand a pinned staging buffer back with the event of the copy that reads it (the
        pool owns the event from then on and waits on it before lending the buffer again);
        otherwise destroy that event."""
        if rec.resident:
            return
        if rec.staged is not rec.host and self._pinned_pool is not None:
            self._pinned_pool.release(rec.staged, copy_event=rec.copied)
        else:
            self.backend.destroy_event(rec.copied)

    # -- one layer's transfer --
    def _issue(self, index: int, layer_id: int, metrics: RuntimeMetrics) -> _Inflight:
        layer = self.layers[layer_id]
        lm = LayerMetrics(layer_id=layer_id)
        t_stall = time.perf_counter()
        self.storage.wait(layer_id)
        host = self.storage.get(layer_id)
        lm.stall_ms = (time.perf_counter() - t_stall) * 1000
        if hasattr(self.storage, "get_disk_read_ms"):
            lm.disk_read_ms = self.storage.get_disk_read_ms(layer_id)
        if self.dequantizer is not None and self.dequantizer.needs_dequantize(layer):
            compressed = host.nbytes
            host = self.dequantizer.dequantize(layer, host)
            lm.compressed_nbytes = compressed
            metrics.compressed_bytes += compressed
        if isinstance(host, DeviceBuffer):
            # a layer resident on the device (DeviceResidentStorage): nothing to copy
            return _Inflight(index, layer, lm, host, host, host, None, resident=True)
        nbytes = host.nbytes
        is_moe = getattr(self.executor, "is_moe_layer", None)
        granular = self.expert_granular and (is_moe(layer) if is_moe is not None else
                                             bool(layer.metadata.get("is_moe", False)))
        staged = host if granular else self._stage_pinned(host)
        device = self._alloc_device(nbytes)
        t0 = time.perf_counter()
        t_start = t_end = None
        if self._timing:
            t_start = self.backend.create_timing_event()
            self.backend.record(t_start, self.transfer_stream)
        if granular:
            core, _ = self.executor.expert_ranges(layer)
            nbytes = self._copy_ranges(device, staged, core)
        else:
            self.backend.copy_h2d_async(device, staged, self.transfer_stream)
        if self._timing:
            t_end = self.backend.create_timing_event()
            self.backend.record(t_end, self.transfer_stream)
        copied = self.backend.record_event(self.transfer_stream)
        elapsed = time.perf_counter() - t0
        lm.h2d_ms = elapsed * 1000
        lm.nbytes = nbytes
        metrics.transfer_seconds += elapsed
        metrics.transferred_bytes += nbytes
        return _Inflight(index, layer, lm, host, staged, device, copied, t_start, t_end,
                         granular)

    def _copy_ranges(self, device: DeviceBuffer, host: HostBuffer,
                     ranges: list[tuple[int, int]]) -> int:
        """H2D of byte ranges of a layer into the same offsets of its device buffer, on
        the transfer stream; returns the bytes enqueued."""
        import numpy as np

        base = int(np.frombuffer(host.view, dtype=np.uint8).ctypes.data)
        total = 0
        for a, b in ranges:
            if b > a:
                self.backend.copy_h2d_ptr_async(int(device.handle) + a, base + a, b - a,
                                                self.transfer_stream)
                total += b - a
        return total

    def _fetch_experts(self, rec: "_Inflight", ids: list[int], metrics: RuntimeMetrics) -> None:
        """Copy the routed experts ``ids`` of an in-flight layer and make the compute
        stream wait for them."""
        _, per_expert = self.executor.expert_ranges(rec.layer)
        t0 = time.perf_counter()
        ev_a = ev_b = None
        if self._timing:
            ev_a = self.backend.create_timing_event()
            self.backend.record(ev_a, self.transfer_stream)
        n = self._copy_ranges(rec.device, rec.staged, [per_expert[e] for e in ids])
        if self._timing:
            ev_b = self.backend.create_timing_event()
            self.backend.record(ev_b, self.transfer_stream)
        done = self.backend.record_event(self.transfer_stream)
        self.backend.wait_event(self.compute_stream, done)
        self.backend.destroy_event(done)
        elapsed = time.perf_counter() - t0
        rec.lm.h2d_ms += elapsed * 1000
        rec.lm.nbytes += n
        metrics.transfer_seconds += elapsed
        metrics.transferred_bytes += n
        if ev_a is not None:
            rec.extra_copies.append((ev_a, ev_b))

    def run_inference(self, ordered_layer_ids: list[int], inputs: Any) -> tuple[Any, RuntimeMetrics]:
        unknown = [lid for lid in ordered_layer_ids if lid not in self.layers]
        if unknown:
            raise ValueError(f"Unknown layer IDs: {unknown}")
        metrics = RuntimeMetrics(layer_count=len(ordered_layer_ids))
        activations = inputs
        wall_start = time.perf_counter()
        for layer_id in self.scheduler.warmup_prefetch_ids(ordered_layer_ids):
            self.storage.request(layer_id)

        inflight: deque[_Inflight] = deque()
        timings: list[tuple[LayerMetrics, Any, Any, Any, Any]] = []
        n = len(ordered_layer_ids)
        next_issue = 0
        try:
            for index, layer_id in enumerate(ordered_layer_ids):
                last = min(n - 1, index + self.transfer_lookahead)
                while next_issue <= last:
                    inflight.append(self._issue(next_issue, ordered_layer_ids[next_issue], metrics))
                    next_issue += 1
                rec = inflight.popleft()
                if rec.copied is not None:
                    self.backend.wait_event(self.compute_stream, rec.copied)

                c_start = c_end = None
                if self._timing:
                    c_start = self.backend.create_timing_event()
                    self.backend.record(c_start, self.compute_stream)
                t1 = time.perf_counter()
                if rec.granular:
                    activations = self.executor.run_layer_granular(
                        layer=rec.layer,
                        activations=activations,
                        device_weights=rec.device,
                        backend=self.backend,
                        stream=self.compute_stream,
                        fetch=lambda ids, rec=rec: self._fetch_experts(rec, ids, metrics),
                    )
                else:
                    activations = self.executor.run_layer(
                        layer=rec.layer,
                        activations=activations,
                        device_weights=rec.device,
                        backend=self.backend,
                        stream=self.compute_stream,
                    )
                compute_elapsed = time.perf_counter() - t1
                if self._timing:
                    c_end = self.backend.create_timing_event()
                    self.backend.record(c_end, self.compute_stream)
                rec.lm.compute_ms = compute_elapsed * 1000
                metrics.compute_seconds += compute_elapsed

                if not rec.resident:
                    # fences the next copy into (or the free of) this layer's buffer
                    done = self.backend.record_event(self.compute_stream)
                    self._free_device(rec.device, done)
                self.storage.release(layer_id)
                self._release_staging(rec)
                timings.append((rec.lm, rec.t_start, rec.t_end, c_start, c_end,
                                rec.extra_copies))
                metrics.layer_metrics.append(rec.lm)
                self._flush_deferred()

                next_layer_id = self.scheduler.next_prefetch_id(ordered_layer_ids, index)
                if next_layer_id is not None:
                    self.storage.request(next_layer_id)
        finally:
            while inflight:
                rec = inflight.popleft()
                self.backend.synchronize_stream(self.transfer_stream)
                if not rec.resident:
                    self._free_device(rec.device, None)
                self._release_staging(rec)
            self.backend.synchronize_stream(self.transfer_stream)
            self.backend.synchronize_stream(self.compute_stream)
            self._flush_deferred(force=True)

        if isinstance(activations, DeviceActivations) and not isinstance(inputs, DeviceActivations):
            # NumPy in, NumPy out (the reference contract); the chain kept them on the device
            activations = activations.numpy()
        metrics.end_to_end_seconds = time.perf_counter() - wall_start
        if self._timing and timings:
            first = None
            for lm, hs, he, cs, ce, extra in timings:
                if hs is not None:
                    lm.h2d_gpu_ms = self.backend.elapsed_ms(hs, he) + \
                        sum(self.backend.elapsed_ms(a, b) for a, b in extra)
                lm.compute_gpu_ms = self.backend.elapsed_ms(cs, ce)
                metrics.transfer_gpu_seconds += lm.h2d_gpu_ms / 1000
                metrics.compute_gpu_seconds += lm.compute_gpu_ms / 1000
                first = (hs if hs is not None else cs) if first is None else first
            metrics.device_seconds = self.backend.elapsed_ms(first, timings[-1][4]) / 1000
            for _, hs, he, cs, ce, extra in timings:
                for ev in (hs, he, cs, ce, *[x for pair in extra for x in pair]):
                    if ev is not None:
                        self.backend.destroy_event(ev)
        return activations, metrics
