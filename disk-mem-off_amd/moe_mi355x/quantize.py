"""Weight formats: per-row symmetric int8 for experts, and the runtime's host dequantizers.

Per-row int8 (fused on the device by the expert kernels): for each output row r of an
nn.Linear weight W [out, in]
    scale[r] = float16(max_c |W[r, c]| / 127)        (1 when the row is all zero or the
                                                      fp16 scale underflows to 0)
    q[r, c]  = clip(rint(W[r, c] / float32(scale[r])), -127, 127)   as int8
    W'[r, c] = q[r, c] * scale[r]
This is the zero-point-0, per-row-scale case of the reference dequantisation formula
``(q - zero_point) * scale`` (offload_runtime/quantize.py:44), which the reference applies
with one scalar scale per layer on the host before the copy.

``Int8Dequantizer`` / ``Float16Dequantizer`` / ``CompositeDequantizer`` keep the runtime's
host dequantisation hook (offload_runtime/quantize.py:14-97, runtime.py:147-151).  A layer
carrying per-row int8 experts must not set ``metadata["dtype"] = "int8"``: that key asks
the runtime to expand the whole layer to fp32 on the host.
"""
from __future__ import annotations

import re
from typing import Any, Protocol

import numpy as np

from .types import HostBuffer, LayerSpec


def quantize_rows_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8 quantisation of a 2-D weight (fp32 or fp16)."""
    w32 = np.asarray(w, dtype=np.float32)
    if w32.ndim != 2:
        raise ValueError("expected a 2-D [out, in] weight")
    amax = np.max(np.abs(w32), axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float16)
    bad = (amax == 0) | (scale == 0)
    scale[bad] = np.float16(1.0)
    q = np.rint(w32 / scale.astype(np.float32)[:, None])
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, scale


def dequantize_rows_int8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return q.astype(np.float32) * np.asarray(scale, dtype=np.float32)[:, None]


_EXPERT_W = re.compile(r"^mlp\.(experts\.\d+|shared_experts?)\.(gate|up|down)_proj\.weight$")


def quantize_moe_tensors(tensors: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    """Offline tool: replace every routed / shared expert projection by int8 + fp16
    per-row scales (``<name>_scale``); other tensors are kept as they are."""
    out: dict[str, np.ndarray] = {}
    for name, arr in tensors.items():
        if _EXPERT_W.match(name):
            q, s = quantize_rows_int8(arr)
            out[name] = q
            out[name + "_scale"] = s
        else:
            out[name] = arr
    return out


class Dequantizer(Protocol):
    def needs_dequantize(self, layer: LayerSpec) -> bool: ...

    def dequantize(self, layer: LayerSpec, buf: HostBuffer) -> HostBuffer: ...

    def decompressed_nbytes(self, layer: LayerSpec) -> int: ...


class Int8Dequantizer:
    """Whole-layer int8 -> fp32 with ``metadata["scale"]`` / ``["zero_point"]``."""

    def needs_dequantize(self, layer: LayerSpec) -> bool:
        return layer.metadata.get("dtype") == "int8"

    def decompressed_nbytes(self, layer: LayerSpec) -> int:
        return layer.nbytes * 4

    def dequantize(self, layer: LayerSpec, buf: HostBuffer) -> HostBuffer:
        scale = layer.metadata.get("scale", 1.0)
        zero_point = layer.metadata.get("zero_point", 0)
        q = np.frombuffer(buf.view, dtype=np.int8)
        out = (q.astype(np.float32) - zero_point) * scale
        return HostBuffer(view=memoryview(bytearray(out.astype(np.float32).tobytes())),
                          pinned=False)


class Float16Dequantizer:
    """Whole-layer fp16 -> fp32."""

    def needs_dequantize(self, layer: LayerSpec) -> bool:
        return layer.metadata.get("dtype") == "float16"

    def decompressed_nbytes(self, layer: LayerSpec) -> int:
        return layer.nbytes * 2

    def dequantize(self, layer: LayerSpec, buf: HostBuffer) -> HostBuffer:
        out = np.frombuffer(buf.view, dtype=np.float16).astype(np.float32)
        return HostBuffer(view=memoryview(bytearray(out.tobytes())), pinned=False)


class CompositeDequantizer:
    """First dequantizer that claims the layer wins; otherwise pass through."""

    def __init__(self, dequantizers: list[Any] | None = None) -> None:
        self._dequantizers = dequantizers or [Int8Dequantizer(), Float16Dequantizer()]

    def needs_dequantize(self, layer: LayerSpec) -> bool:
        return any(d.needs_dequantize(layer) for d in self._dequantizers)

    def decompressed_nbytes(self, layer: LayerSpec) -> int:
        for d in self._dequantizers:
            if d.needs_dequantize(layer):
                return d.decompressed_nbytes(layer)
        return layer.nbytes

    def dequantize(self, layer: LayerSpec, buf: HostBuffer) -> HostBuffer:
        for d in self._dequantizers:
            if d.needs_dequantize(layer):
                return d.dequantize(layer, buf)
        return buf
