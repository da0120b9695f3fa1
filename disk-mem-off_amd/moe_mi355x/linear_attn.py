"""Qwen3-Next linear-attention (Gated DeltaNet) block on the MI355X.

Device counterpart of ``Qwen3NextExecutor._linear_attn_block``
(offload_runtime/executors/qwen3_next.py:207-269) through ``mx_linear_attn_forward``.  The
block reads its tensors in place from a packed layer buffer (``LinearAttnLayout`` resolves
the ``linear_attn.*`` / ``input_layernorm.weight`` entries of ``layer.metadata["tensors"]``),
so a layer's attention weights never travel back to the host.

The reference reshapes q and k with the value-head count (qwen3_next.py:75-77), so it runs
only when ``linear_num_key_heads == linear_num_value_heads``; the same condition is
enforced here with a ``ValueError``.  The recurrent state starts at zero on every call,
as in the reference.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import numpy as np

from . import _lib
from .types import DeviceBuffer

IN_NORM = "input_layernorm.weight"
QKVZ = "linear_attn.in_proj_qkvz.weight"
BA = "linear_attn.in_proj_ba.weight"
CONV = "linear_attn.conv1d.weight"
A_LOG = "linear_attn.A_log"
DT_BIAS = "linear_attn.dt_bias"
OUT_NORM = "linear_attn.norm.weight"
OUT = "linear_attn.out_proj.weight"
NAMES = (IN_NORM, QKVZ, BA, CONV, A_LOG, DT_BIAS, OUT_NORM, OUT)

_DT = {"float32": _lib.MX_DT_F32, "float16": _lib.MX_DT_F16, "int8": _lib.MX_DT_I8}


def has_linear_attn(meta: list[dict[str, Any]]) -> bool:
    return any(m["name"].startswith("linear_attn.") for m in meta)


@dataclass(frozen=True)
class LinearAttnLayout:
    """Shapes, element types and byte offsets of a packed layer's linear-attention tensors."""

    hidden: int
    n_heads: int
    head_dim_k: int
    head_dim_v: int
    conv_kernel: int
    weight_dtype: int
    param_dtype: int
    offsets: dict[str, int]

    @classmethod
    def from_meta(cls, meta: list[dict[str, Any]]) -> "LinearAttnLayout":
        by = {m["name"]: m for m in meta}
        missing = [n for n in NAMES if n not in by]
        if missing:
            raise ValueError(f"layer lacks linear-attention tensors {missing}")
        n = int(by[A_LOG]["shape"][0])
        H = int(by[IN_NORM]["shape"][0])
        ba_rows, ba_in = (int(v) for v in by[BA]["shape"])
        qkvz_rows, qkvz_in = (int(v) for v in by[QKVZ]["shape"])
        if (ba_rows - n) % n or ba_in != H or qkvz_in != H:
            raise ValueError(f"in_proj_ba {by[BA]['shape']} does not fit {n} heads of hidden {H}")
        dk = (ba_rows - n) // n
        vd2 = qkvz_rows - 2 * n * dk
        if vd2 <= 0 or vd2 % (2 * n):
            raise ValueError(f"in_proj_qkvz {by[QKVZ]['shape']} does not fit {n} heads x {dk}")
        dv = vd2 // (2 * n)
        conv_shape = [int(v) for v in by[CONV]["shape"]]
        if conv_shape[0] != n * (2 * dk + dv) or (len(conv_shape) == 3 and conv_shape[1] != 1):
            raise ValueError(f"conv1d weight {conv_shape} does not fit the projections")
        if [int(v) for v in by[OUT]["shape"]] != [H, n * dv] or \
                [int(v) for v in by[OUT_NORM]["shape"]] != [n * dv] or \
                [int(v) for v in by[DT_BIAS]["shape"]] != [n]:
            raise ValueError("out_proj / norm / dt_bias shapes do not fit the projections")
        wdts = {by[k]["dtype"] for k in (QKVZ, BA, OUT)}
        pdts = {by[k]["dtype"] for k in (IN_NORM, CONV, A_LOG, DT_BIAS, OUT_NORM)}
        if len(wdts) != 1 or len(pdts) != 1:
            raise ValueError(f"mixed element types: projections {wdts}, parameters {pdts}")
        wdt, pdt = _DT.get(wdts.pop()), _DT.get(pdts.pop())
        if wdt is None or pdt is None or pdt == _lib.MX_DT_I8:
            raise ValueError("projections must be float32/float16/int8 and parameters "
                             "float32/float16")
        offsets = {k: int(by[k]["offset"]) for k in NAMES}
        if wdt == _lib.MX_DT_I8:
            for k in (QKVZ, BA, OUT):
                if k + "_scale" not in by:
                    raise ValueError(f"int8 {k} has no {k}_scale")
                offsets[k + "_scale"] = int(by[k + "_scale"]["offset"])
        return cls(H, n, dk, dv, conv_shape[-1], wdt, pdt, offsets)

    def desc(self, eps: float) -> _lib.MxLinearAttnDesc:
        return _lib.MxLinearAttnDesc(self.hidden, self.n_heads, self.head_dim_k, self.head_dim_v,
                                     self.conv_kernel, self.weight_dtype, self.param_dtype,
                                     float(eps))

    def weights(self, base: int) -> _lib.MxLinearAttnWeights:
        o = self.offsets

        def at(name: str) -> int | None:
            return base + o[name] if name in o else None

        return _lib.MxLinearAttnWeights(at(IN_NORM), at(QKVZ), at(QKVZ + "_scale"), at(BA),
                                        at(BA + "_scale"), at(CONV), at(A_LOG), at(DT_BIAS),
                                        at(OUT_NORM), at(OUT), at(OUT + "_scale"))


def workspace_bytes(desc: _lib.MxLinearAttnDesc, tokens: int) -> int:
    n = ctypes.c_size_t()
    _lib.check(_lib.load().mx_linear_attn_workspace_size(ctypes.byref(desc), tokens,
                                                         ctypes.byref(n)),
               "mx_linear_attn_workspace_size")
    return int(n.value)


class LinearAttnRunner:
    """Workspace and host staging for linear-attention blocks on one stream."""

    def __init__(self, backend: Any) -> None:
        self.backend = backend
        self.lib = _lib.load()
        self._ws: DeviceBuffer | None = None
        self._io: dict[str, DeviceBuffer] = {}
        self._pinned: dict[str, Any] = {}

    def reserve(self, desc: _lib.MxLinearAttnDesc, tokens: int, io: bool = True) -> None:
        need = workspace_bytes(desc, tokens)
        if self._ws is None or self._ws.nbytes < need:
            if self._ws is not None:
                self.backend.free_device(self._ws)
            self._ws = self.backend.alloc_device(need)
        if not io:
            return
        nb = max(tokens * desc.hidden * 4, 16)
        for key in ("x", "out"):
            buf = self._io.get(key)
            if buf is None or buf.nbytes < nb:
                if buf is not None:
                    self.backend.free_device(buf)
                self._io[key] = self.backend.alloc_device(nb)
            pin = self._pinned.get(key)
            if pin is None or pin.nbytes < nb:
                if pin is not None:
                    self.backend.free_pinned_host(pin)
                self._pinned[key] = self.backend.alloc_pinned_host(nb)

    def forward_device(self, desc: _lib.MxLinearAttnDesc, weights: _lib.MxLinearAttnWeights,
                       x: int, out: int, tokens: int, stream: Any,
                       events: list[int] | None = None) -> None:
        """out[T, H] = x + linear attention(x); device pointers; asynchronous."""
        ws = self._ws
        if ws is None:
            raise RuntimeError("LinearAttnRunner.reserve() must run before forward_device()")
        if events is None:
            rc = self.lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(weights), x,
                                                 out, tokens, ws.handle, ws.nbytes, stream)
        else:
            arr = (ctypes.c_void_p * len(events))(*events)
            rc = self.lib.mx_linear_attn_forward_profiled(ctypes.byref(desc),
                                                          ctypes.byref(weights), x, out, tokens,
                                                          ws.handle, ws.nbytes, stream, arr,
                                                          len(events))
        _lib.check(rc, "mx_linear_attn_forward")

    def forward_numpy(self, desc: _lib.MxLinearAttnDesc, weights: _lib.MxLinearAttnWeights,
                      x: np.ndarray, stream: Any) -> np.ndarray:
        """Host fp32 [T, H] in and out; synchronises ``stream``."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != desc.hidden:
            raise ValueError(f"activations must be [T, {desc.hidden}], got {x.shape}")
        T = x.shape[0]
        if T == 0:
            return x.copy()
        self.reserve(desc, T)
        px, po = self._pinned["x"], self._pinned["out"]
        np.frombuffer(px.view, dtype=np.uint8, count=x.nbytes)[:] = x.view(np.uint8).ravel()
        ax = ctypes.addressof(ctypes.c_char.from_buffer(px.view))
        ao = ctypes.addressof(ctypes.c_char.from_buffer(po.view))
        self.backend.copy_h2d_ptr_async(self._io["x"].handle, ax, x.nbytes, stream)
        self.forward_device(desc, weights, self._io["x"].handle, self._io["out"].handle, T,
                            stream)
        self.backend.copy_d2h_ptr_async(ao, self._io["out"].handle, x.nbytes, stream)
        self.backend.synchronize_stream(stream)
        return np.frombuffer(po.view, dtype=np.float32, count=x.size).reshape(x.shape).copy()

    def views(self, desc: _lib.MxLinearAttnDesc, tokens: int) -> _lib.MxLinearAttnViews:
        if self._ws is None:
            raise RuntimeError("no workspace reserved")
        v = _lib.MxLinearAttnViews()
        _lib.check(self.lib.mx_linear_attn_views(ctypes.byref(desc), tokens, self._ws.handle,
                                                 ctypes.byref(v)), "mx_linear_attn_views")
        return v

    def close(self) -> None:
        if self._ws is not None:
            self.backend.free_device(self._ws)
            self._ws = None
        for buf in self._io.values():
            self.backend.free_device(buf)
        self._io.clear()
        for pin in self._pinned.values():
            self.backend.free_pinned_host(pin)
        self._pinned.clear()


class DeviceLinearAttnLayer:
    """A linear-attention block resident in HBM (packed like a loader layer, 16-byte
    aligned tensors) with the runner that executes it."""

    def __init__(self, backend: Any, buf: DeviceBuffer, meta: list[dict[str, Any]],
                 stream: Any) -> None:
        self.backend = backend
        self.buf = buf
        self.meta = meta
        self.stream = stream
        self.layout = LinearAttnLayout.from_meta(meta)
        self.runner = LinearAttnRunner(backend)

    @classmethod
    def from_host(cls, backend: Any, tensors: dict[str, np.ndarray],
                  stream: Any) -> "DeviceLinearAttnLayer":
        from .layout import pack_tensors

        raw, meta = pack_tensors(tensors, align=16)
        buf = backend.alloc_device(max(len(raw), 16))
        pin = backend.alloc_pinned_host(max(len(raw), 16))
        try:
            np.frombuffer(pin.view, dtype=np.uint8, count=len(raw))[:] = np.frombuffer(
                raw, dtype=np.uint8)
            backend.copy_h2d_ptr_async(buf.handle,
                                       ctypes.addressof(ctypes.c_char.from_buffer(pin.view)),
                                       len(raw), stream)
            backend.synchronize_stream(stream)
        finally:
            backend.free_pinned_host(pin)
        return cls(backend, buf, meta, stream)

    def desc(self, eps: float) -> _lib.MxLinearAttnDesc:
        return self.layout.desc(eps)

    def weights(self) -> _lib.MxLinearAttnWeights:
        return self.layout.weights(int(self.buf.handle))

    def forward_numpy(self, x: np.ndarray, eps: float) -> np.ndarray:
        return self.runner.forward_numpy(self.desc(eps), self.weights(), x, self.stream)

    def close(self) -> None:
        self.runner.close()
        if self.buf is not None:
            self.backend.free_device(self.buf)
            self.buf = None
