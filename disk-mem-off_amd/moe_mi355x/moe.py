"""Host driver of the device MoE block: configuration, workspace, pointer tables, I/O.

``MoeConfig`` carries the executor config keys of the reference (glm4_moe.py:70-84,
qwen3_next.py:126-133) plus the two choices the reference does not expose: the router
mode and the expert weight format.  ``MoeRunner`` owns the device workspace, the expert
pointer table and pinned staging for NumPy inputs/outputs, and calls ``mx_moe_forward``.
All allocation happens in ``reserve``/``bind``; ``forward_device`` allocates nothing.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from . import _lib
from .backends import MI355XBackend
from .layout import MoeLayerLayout
from .types import DeviceBuffer

ROUTER_MODES = {
    "ref_softmax_bias": _lib.MX_ROUTER_REF_SOFTMAX_BIAS,
    "sigmoid_select_bias": _lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
    "softmax": _lib.MX_ROUTER_SOFTMAX,
}


@dataclass
class MoeConfig:
    hidden: int
    inter: int
    shared_inter: int
    n_experts: int
    top_k: int
    router_mode: int
    norm_topk_prob: bool
    routed_scaling: float
    eps: float
    weight_dtype: int
    param_dtype: int
    has_bias: bool
    has_shared_gate: bool
    weight_layout: int = _lib.MX_LAYOUT_ROWS

    @classmethod
    def from_layout(cls, layout: MoeLayerLayout, *, top_k: int, router_mode: int | str,
                    norm_topk_prob: bool, routed_scaling: float, eps: float,
                    weight_layout: int = _lib.MX_LAYOUT_ROWS) -> "MoeConfig":
        if isinstance(router_mode, str):
            router_mode = ROUTER_MODES[router_mode]
        return cls(hidden=layout.hidden, inter=layout.inter, shared_inter=layout.shared_inter,
                   n_experts=layout.n_experts, top_k=top_k, router_mode=router_mode,
                   norm_topk_prob=bool(norm_topk_prob), routed_scaling=float(routed_scaling),
                   eps=float(eps), weight_dtype=layout.weight_dtype,
                   param_dtype=layout.param_dtype,
                   has_bias=layout.has_bias and router_mode != _lib.MX_ROUTER_SOFTMAX,
                   has_shared_gate=layout.has_shared_gate, weight_layout=int(weight_layout))

    def desc(self) -> _lib.MxMoeDesc:
        return _lib.MxMoeDesc(
            hidden=self.hidden, inter=self.inter, shared_inter=self.shared_inter,
            n_experts=self.n_experts, top_k=self.top_k, router_mode=self.router_mode,
            norm_topk_prob=int(self.norm_topk_prob), weight_dtype=self.weight_dtype,
            param_dtype=self.param_dtype, has_bias=int(self.has_bias),
            has_shared_gate=int(self.has_shared_gate), routed_scaling=self.routed_scaling,
            eps=self.eps, weight_layout=self.weight_layout)


_ELEM = {_lib.MX_DT_F32: 4, _lib.MX_DT_F16: 2, _lib.MX_DT_I8: 1}


def tile_experts(backend: Any, layout: MoeLayerLayout, base: int, stream: Any) -> None:
    """Re-lay every expert matrix of the layer at device address ``base`` from the loader's
    row-major form into MX_LAYOUT_FRAG16, in place (through one scratch matrix).  Raises
    ``ValueError`` when a shape has no whole fragments (rows % 16, cols % (64 / size))."""
    lib = _lib.load()
    esz = _ELEM[layout.weight_dtype]
    mats = layout.expert_matrices()
    for _, r, c in mats:
        if r % 16 or (c * esz) % 64:
            raise ValueError(f"expert matrix {r}x{c} has no whole 16 x {64 // esz} fragments")
    scratch = backend.alloc_device(max(r * c * esz for _, r, c in mats))
    try:
        for off, r, c in mats:
            _lib.check(lib.mx_memcpy_d2d_async(scratch.handle, base + off, r * c * esz, stream),
                       "hipMemcpyAsync")
            _lib.check(lib.mx_tile_weights(base + off, scratch.handle, r, c,
                                           layout.weight_dtype, stream), "mx_tile_weights")
        backend.synchronize_stream(stream)
    finally:
        backend.free_device(scratch)


def workspace_bytes(desc: _lib.MxMoeDesc, tokens: int) -> int:
    n = ctypes.c_size_t()
    _lib.check(_lib.load().mx_moe_workspace_size(ctypes.byref(desc), tokens, ctypes.byref(n)),
               "mx_moe_workspace_size")
    return int(n.value)


class MoeRunner:
    """Device resources for running MoE blocks of one shape family on one stream."""

    def __init__(self, backend: MI355XBackend) -> None:
        self.backend = backend
        self.lib = _lib.load()
        self._ws: DeviceBuffer | None = None
        self._table_dev: DeviceBuffer | None = None
        # The layout object and buffer address the uploaded pointer table was built from;
        # the layout is held by reference so a new layout can never be taken for it.
        self._table_layout: MoeLayerLayout | None = None
        self._table_base: int | None = None
        self._table_ev: Any = None
        self._io: dict[str, DeviceBuffer] = {}
        self._pinned: dict[str, Any] = {}
        self._split_tokens = 0

    # -- allocation (never called from forward_device) --
    def reserve(self, desc: _lib.MxMoeDesc, tokens: int) -> None:
        need = workspace_bytes(desc, tokens)
        if self._ws is None or self._ws.nbytes < need:
            if self._ws is not None:
                self.backend.free_device(self._ws)
            self._ws = self.backend.alloc_device(need)
        nbytes_act = tokens * desc.hidden * 4
        for key in ("x", "out"):
            buf = self._io.get(key)
            if buf is None or buf.nbytes < nbytes_act:
                if buf is not None:
                    self.backend.free_device(buf)
                self._io[key] = self.backend.alloc_device(max(nbytes_act, 16))
            pin = self._pinned.get(key)
            if pin is None or pin.nbytes < nbytes_act:
                if pin is not None:
                    self.backend.free_pinned_host(pin)
                self._pinned[key] = self.backend.alloc_pinned_host(max(nbytes_act, 16))

    def bind(self, layout: MoeLayerLayout, base: int, stream: Any) -> _lib.MxMoeWeights:
        """Upload the expert pointer table for a layer buffer at ``base`` (cached while the
        same layout object is bound at the same address)."""
        nbytes = ctypes.sizeof(_lib.MxExpertPtrs) * (layout.n_experts + 1)
        if self._table_dev is None or self._table_dev.nbytes < nbytes:
            self._wait_table_upload()
            if self._table_dev is not None:
                self.backend.free_device(self._table_dev)
            self._table_dev = self.backend.alloc_device(nbytes)
            self._table_layout = self._table_base = None
            pin = self._pinned.pop("table", None)
            if pin is not None:
                self.backend.free_pinned_host(pin)
            self._pinned["table"] = self.backend.alloc_pinned_host(nbytes)
        if self._table_layout is not layout or self._table_base != base:
            table = layout.expert_table(base)
            pin = self._pinned["table"]
            # The previous upload may still be reading the pinned staging copy.
            self._wait_table_upload()
            ctypes.memmove(ctypes.addressof(ctypes.c_char.from_buffer(pin.view)), table, nbytes)
            self.backend.copy_h2d_ptr_async(self._table_dev.handle,
                                            ctypes.addressof(ctypes.c_char.from_buffer(pin.view)),
                                            nbytes, stream)
            self._table_ev = self.backend.record_event(stream)
            self._table_layout, self._table_base = layout, base
        return layout.weights(base, self._table_dev.handle)

    def _wait_table_upload(self) -> None:
        if self._table_ev is not None:
            sync = getattr(self.backend, "event_synchronize", None)
            if sync is not None:
                sync(self._table_ev)
            self.backend.destroy_event(self._table_ev)
            self._table_ev = None

    # -- hot path --
    def forward_device(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, x: int, out: int,
                       tokens: int, stream: Any, events: list[int] | None = None) -> None:
        """out[T, H] = MoE block(x[T, H]); device pointers; asynchronous on ``stream``."""
        ws = self._ws
        if ws is None:
            raise RuntimeError("MoeRunner.reserve() must run before forward_device()")
        if events is None:
            rc = self.lib.mx_moe_forward(ctypes.byref(desc), ctypes.byref(weights), x, out,
                                         tokens, ws.handle, ws.nbytes, stream)
        else:
            arr = (ctypes.c_void_p * len(events))(*events)
            rc = self.lib.mx_moe_forward_profiled(ctypes.byref(desc), ctypes.byref(weights), x,
                                                  out, tokens, ws.handle, ws.nbytes, stream,
                                                  arr, len(events))
        _lib.check(rc, "mx_moe_forward")

    def forward_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, x: np.ndarray,
                      stream: Any, pre: Callable[[int, int], None] | None = None) -> np.ndarray:
        """Host fp32 [T, H] in, host fp32 [T, H] out; synchronises ``stream``.  ``pre(x_dev,
        T)``, when given, runs on ``stream`` after the upload and rewrites the device copy of
        x in place (for example the layer's attention block) before the MoE block reads it."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != desc.hidden:
            raise ValueError(f"activations must be [T, {desc.hidden}], got {x.shape}")
        T = x.shape[0]
        self.reserve(desc, max(T, 1))
        if T == 0:
            return x.copy()
        nb = x.nbytes
        px, po = self._pinned["x"], self._pinned["out"]
        np.frombuffer(px.view, dtype=np.uint8, count=nb)[:] = x.view(np.uint8).ravel()
        addr_x = ctypes.addressof(ctypes.c_char.from_buffer(px.view))
        addr_o = ctypes.addressof(ctypes.c_char.from_buffer(po.view))
        self.backend.copy_h2d_ptr_async(self._io["x"].handle, addr_x, nb, stream)
        if pre is not None:
            pre(self._io["x"].handle, T)
        self.forward_device(desc, weights, self._io["x"].handle, self._io["out"].handle, T, stream)
        self.backend.copy_d2h_ptr_async(addr_o, self._io["out"].handle, nb, stream)
        self.backend.synchronize_stream(stream)
        return np.frombuffer(po.view, dtype=np.float32, count=T * desc.hidden).reshape(T, -1).copy()

    # -- split forward (router part, then the expert part after the experts are copied) --
    def route_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, x: np.ndarray,
                    stream: Any, pre: Callable[[int, int], None] | None = None) -> list[int]:
        """Upload x (then ``pre`` as in ``forward_numpy``) and run stages 0..3 (RMSNorm,
        router, top-k, dispatch); returns the routed experts the batch uses, ascending
        (synchronises ``stream``)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != desc.hidden:
            raise ValueError(f"activations must be [T, {desc.hidden}], got {x.shape}")
        T = x.shape[0]
        self.reserve(desc, max(T, 1))
        self._split_tokens = T
        if T == 0:
            return []
        px = self._pinned["x"]
        np.frombuffer(px.view, dtype=np.uint8, count=x.nbytes)[:] = x.view(np.uint8).ravel()
        self.backend.copy_h2d_ptr_async(self._io["x"].handle,
                                        ctypes.addressof(ctypes.c_char.from_buffer(px.view)),
                                        x.nbytes, stream)
        if pre is not None:
            pre(self._io["x"].handle, T)
        self._stages(desc, weights, T, 0, _lib.MX_STAGE_ROUTE_END, stream)
        v = self.views(desc, T)
        ng = int(read_device(self.backend, v.n_groups, np.int32, 1, stream)[0])
        ge = read_device(self.backend, v.g_expert, np.int32, ng, stream)
        return sorted(int(e) for e in ge if e < desc.n_experts)

    def finish_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights,
                     stream: Any) -> np.ndarray:
        """Stages 4..6 for the batch of the last ``route_numpy``; synchronises ``stream``."""
        T = self._split_tokens
        nb = T * desc.hidden * 4
        if T == 0:
            return np.zeros((0, desc.hidden), np.float32)
        self._stages(desc, weights, T, _lib.MX_STAGE_ROUTE_END, _lib.MX_N_STAGES, stream)
        po = self._pinned["out"]
        addr_o = ctypes.addressof(ctypes.c_char.from_buffer(po.view))
        self.backend.copy_d2h_ptr_async(addr_o, self._io["out"].handle, nb, stream)
        self.backend.synchronize_stream(stream)
        return np.frombuffer(po.view, dtype=np.float32, count=T * desc.hidden).reshape(T, -1).copy()

    def _stages(self, desc, weights, T: int, begin: int, end: int, stream: Any) -> None:
        ws = self._ws
        _lib.check(self.lib.mx_moe_forward_stages(ctypes.byref(desc), ctypes.byref(weights),
                                                  self._io["x"].handle, self._io["out"].handle,
                                                  T, ws.handle, ws.nbytes, begin, end, stream),
                   "mx_moe_forward_stages")

    # -- inspection --
    def views(self, desc: _lib.MxMoeDesc, tokens: int) -> _lib.MxMoeViews:
        v = _lib.MxMoeViews()
        _lib.check(self.lib.mx_moe_views(ctypes.byref(desc), tokens, self._ws.handle,
                                         ctypes.byref(v)), "mx_moe_views")
        return v

    def close(self) -> None:
        self._wait_table_upload()
        for buf in [self._ws, self._table_dev, *self._io.values()]:
            if buf is not None:
                self.backend.free_device(buf)
        for pin in self._pinned.values():
            self.backend.free_pinned_host(pin)
        self._ws = self._table_dev = None
        self._table_layout = self._table_base = None
        self._io.clear()
        self._pinned.clear()


def read_device(backend: MI355XBackend, ptr: int, dtype: Any, count: int, stream: Any = None) -> np.ndarray:
    """Synchronous copy of ``count`` elements at a device address into a new array."""
    out = np.empty(count, dtype=dtype)
    if count:
        backend.copy_d2h_ptr_async(out.ctypes.data, ptr, out.nbytes, stream)
        backend.synchronize_stream(stream)
    return out
