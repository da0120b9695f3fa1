"""Qwen3-Next gated full-attention block on the MI355X.

Device counterpart of ``Qwen3NextExecutor._full_attn_block``
(offload_runtime/executors/qwen3_next.py:161-205) through ``mx_full_attn_forward``.  The
block reads its tensors in place from a packed layer buffer (``FullAttnLayout`` resolves the
``self_attn.*`` / ``input_layernorm.weight`` entries of ``layer.metadata["tensors"]``).
Head counts, head_dim and the rotary size come from the executor config, as in the
reference (qwen3_next.py:106-118); the tensor shapes are checked against them.  There is no
KV cache: each call attends over its own tokens at positions 0 .. T-1, as in the reference.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import numpy as np

from . import _lib
from .types import DeviceBuffer

IN_NORM = "input_layernorm.weight"
Q = "self_attn.q_proj.weight"
K = "self_attn.k_proj.weight"
V = "self_attn.v_proj.weight"
O = "self_attn.o_proj.weight"
Q_NORM = "self_attn.q_norm.weight"
K_NORM = "self_attn.k_norm.weight"

_DT = {"float32": _lib.MX_DT_F32, "float16": _lib.MX_DT_F16, "int8": _lib.MX_DT_I8}


def has_full_attn(meta: list[dict[str, Any]]) -> bool:
    return any(m["name"] == Q for m in meta)


@dataclass(frozen=True)
class FullAttnLayout:
    """Shapes, element types and byte offsets of a packed layer's attention tensors."""

    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rotary_dim: int
    rope_theta: float
    weight_dtype: int
    param_dtype: int
    offsets: dict[str, int]

    @classmethod
    def from_meta(cls, meta: list[dict[str, Any]], n_heads: int, n_kv_heads: int,
                  head_dim: int, rotary_dim: int, rope_theta: float) -> "FullAttnLayout":
        by = {m["name"]: m for m in meta}
        missing = [n for n in (IN_NORM, Q, K, V, O) if n not in by]
        if missing:
            raise ValueError(f"layer lacks attention tensors {missing}")
        H = int(by[IN_NORM]["shape"][0])
        want = {Q: [2 * n_heads * head_dim, H], K: [n_kv_heads * head_dim, H],
                V: [n_kv_heads * head_dim, H], O: [H, n_heads * head_dim]}
        for name, shp in want.items():
            if [int(v) for v in by[name]["shape"]] != shp:
                raise ValueError(f"{name} has shape {by[name]['shape']}, expected {shp} for "
                                 f"{n_heads} heads / {n_kv_heads} kv heads of {head_dim}")
        norms = [n for n in (Q_NORM, K_NORM) if n in by]
        for n in norms:
            if [int(v) for v in by[n]["shape"]] != [head_dim]:
                raise ValueError(f"{n} has shape {by[n]['shape']}, expected [{head_dim}]")
        wdts = {by[k]["dtype"] for k in (Q, K, V, O)}
        pdts = {by[k]["dtype"] for k in [IN_NORM, *norms]}
        if len(wdts) != 1 or len(pdts) != 1:
            raise ValueError(f"mixed element types: projections {wdts}, parameters {pdts}")
        wdt, pdt = _DT.get(wdts.pop()), _DT.get(pdts.pop())
        if wdt is None or pdt is None or pdt == _lib.MX_DT_I8:
            raise ValueError("projections must be float32/float16/int8 and parameters "
                             "float32/float16")
        offsets = {k: int(by[k]["offset"]) for k in [IN_NORM, Q, K, V, O, *norms]}
        if wdt == _lib.MX_DT_I8:
            for k in (Q, K, V, O):
                if k + "_scale" not in by:
                    raise ValueError(f"int8 {k} has no {k}_scale")
                offsets[k + "_scale"] = int(by[k + "_scale"]["offset"])
        return cls(H, n_heads, n_kv_heads, head_dim, rotary_dim, float(rope_theta), wdt, pdt,
                   offsets)

    def desc(self, eps: float) -> _lib.MxFullAttnDesc:
        return _lib.MxFullAttnDesc(self.hidden, self.n_heads, self.n_kv_heads, self.head_dim,
                                   self.rotary_dim, self.weight_dtype, self.param_dtype,
                                   self.rope_theta, float(eps))

    def weights(self, base: int) -> _lib.MxFullAttnWeights:
        o = self.offsets

        def at(name: str) -> int | None:
            return base + o[name] if name in o else None

        return _lib.MxFullAttnWeights(at(IN_NORM), at(Q), at(Q + "_scale"), at(K),
                                      at(K + "_scale"), at(V), at(V + "_scale"), at(O),
                                      at(O + "_scale"), at(Q_NORM), at(K_NORM))


def workspace_bytes(desc: _lib.MxFullAttnDesc, tokens: int) -> int:
    n = ctypes.c_size_t()
    _lib.check(_lib.load().mx_full_attn_workspace_size(ctypes.byref(desc), tokens,
                                                       ctypes.byref(n)),
               "mx_full_attn_workspace_size")
    return int(n.value)


class FullAttnRunner:
    """Workspace and host staging for full-attention blocks on one stream."""

    def __init__(self, backend: Any) -> None:
        self.backend = backend
        self.lib = _lib.load()
        self._ws: DeviceBuffer | None = None
        self._io: dict[str, DeviceBuffer] = {}
        self._pinned: dict[str, Any] = {}

    def reserve(self, desc: _lib.MxFullAttnDesc, tokens: int, io: bool = True) -> None:
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

    def forward_device(self, desc: _lib.MxFullAttnDesc, weights: _lib.MxFullAttnWeights,
                       x: int, out: int, tokens: int, stream: Any,
                       events: list[int] | None = None) -> None:
        """out[T, H] = x + gated attention(x); device pointers; asynchronous."""
        ws = self._ws
        if ws is None:
            raise RuntimeError("FullAttnRunner.reserve() must run before forward_device()")
        if events is None:
            rc = self.lib.mx_full_attn_forward(ctypes.byref(desc), ctypes.byref(weights), x, out,
                                               tokens, ws.handle, ws.nbytes, stream)
        else:
            arr = (ctypes.c_void_p * len(events))(*events)
            rc = self.lib.mx_full_attn_forward_profiled(ctypes.byref(desc),
                                                        ctypes.byref(weights), x, out, tokens,
                                                        ws.handle, ws.nbytes, stream, arr,
                                                        len(events))
        _lib.check(rc, "mx_full_attn_forward")

    def forward_numpy(self, desc: _lib.MxFullAttnDesc, weights: _lib.MxFullAttnWeights,
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

    def views(self, desc: _lib.MxFullAttnDesc, tokens: int) -> _lib.MxFullAttnViews:
        if self._ws is None:
            raise RuntimeError("no workspace reserved")
        v = _lib.MxFullAttnViews()
        _lib.check(self.lib.mx_full_attn_views(ctypes.byref(desc), tokens, self._ws.handle,
                                               ctypes.byref(v)), "mx_full_attn_views")
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


class DeviceFullAttnLayer:
    """A gated full-attention block resident in HBM (packed like a loader layer, 16-byte
    aligned tensors) with the runner that executes it."""

    def __init__(self, backend: Any, buf: DeviceBuffer, layout: FullAttnLayout,
                 stream: Any) -> None:
        self.backend = backend
        self.buf = buf
        self.layout = layout
        self.stream = stream
        self.runner = FullAttnRunner(backend)

    @classmethod
    def from_host(cls, backend: Any, tensors: dict[str, np.ndarray], n_heads: int,
                  n_kv_heads: int, head_dim: int, rotary_dim: int, rope_theta: float,
                  stream: Any) -> "DeviceFullAttnLayer":
        from .layout import pack_tensors

        raw, meta = pack_tensors(tensors, align=16)
        lay = FullAttnLayout.from_meta(meta, n_heads, n_kv_heads, head_dim, rotary_dim,
                                       rope_theta)
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
        return cls(backend, buf, lay, stream)

    def desc(self, eps: float) -> _lib.MxFullAttnDesc:
        return self.layout.desc(eps)

    def weights(self) -> _lib.MxFullAttnWeights:
        return self.layout.weights(int(self.buf.handle))

    def forward_numpy(self, x: np.ndarray, eps: float) -> np.ndarray:
        return self.runner.forward_numpy(self.desc(eps), self.weights(), x, self.stream)

    def close(self) -> None:
        self.runner.close()
        if self.buf is not None:
            self.backend.free_device(self.buf)
            self.buf = None
