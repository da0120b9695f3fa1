"""Host driver of the device MoE block: configuration, workspace, pointer tables, I/O.

``MoeConfig`` carries the executor config keys of the reference (glm4_moe.py:70-84,
qwen3_next.py:126-133) plus the choices the reference does not expose: the router mode,
the expert weight format and layout.  ``MoeRunner`` owns the device workspace, the expert
pointer tables, the device activation buffers and pinned staging for NumPy inputs/outputs,
and calls ``mx_moe_forward``.  Allocation happens in ``reserve`` and at a table's first
``bind``; ``forward_device`` allocates nothing.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from . import _lib
from .activations import DeviceActivations
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
    """Device resources for running MoE blocks of one shape family on one stream.

    * workspace (``reserve``), sized by ``mx_moe_workspace_size``;
    * one expert pointer table per (layer layout, buffer address), uploaded at its first
      ``bind`` and kept (a layer streamed through a pool of k buffers has at most k);
    * activations: an input buffer (NumPy inputs are uploaded into it through pinned
      staging) and two output buffers used in turn, so a layer's output can be handed to the
      next layer on the device (``DeviceActivations``) while that layer writes the other.
    """

    MAX_TABLES = 256
    _SLOTS = ("x", "out", "out2")  # generation-counted device activation buffers

    def __init__(self, backend: MI355XBackend) -> None:
        self.backend = backend
        self.lib = _lib.load()
        self._ws: DeviceBuffer | None = None
        # (id(layout), base) -> (layout, device table, weights struct); the layout is held so
        # its id cannot be reused by another layout while the entry lives.
        self._tables: dict[tuple[int, int], tuple[MoeLayerLayout, DeviceBuffer, Any]] = {}
        self._table_ev: Any = None   # last table upload (reads the pinned staging copy)
        self._x_ev: Any = None       # last upload of x (reads the pinned staging copy)
        self._io: dict[str, DeviceBuffer] = {}
        self._pinned: dict[str, Any] = {}
        self._gen = [0, 0, 0]
        self._next_out = 1
        self._closed = False
        self._last_stream: Any = None
        # tokens, output slot and input address of the last route_numpy
        self._split: tuple[int, int, int] = (0, 1, 0)
        self._reserved: dict[bytes, int] = {}  # desc bytes -> tokens its buffers cover

    def generation(self, slot: int) -> int:
        return -1 if self._closed else self._gen[slot]

    # -- allocation (never called from forward_device) --
    def _quiesce(self) -> None:
        """Wait for the work that may still read buffers about to be freed."""
        if self._last_stream is not None:
            self.backend.synchronize_stream(self._last_stream)

    def reserve(self, desc: _lib.MxMoeDesc, tokens: int) -> None:
        key = bytes(desc)
        if self._reserved.get(key, -1) >= tokens:
            return
        need = workspace_bytes(desc, tokens)
        if self._ws is None or self._ws.nbytes < need:
            self._quiesce()
            if self._ws is not None:
                self.backend.free_device(self._ws)
            self._ws = self.backend.alloc_device(need)
        nbytes_act = tokens * desc.hidden * 4
        for i, key in enumerate(self._SLOTS):
            buf = self._io.get(key)
            if buf is None or buf.nbytes < nbytes_act:
                self._quiesce()
                if buf is not None:
                    self.backend.free_device(buf)
                self._io[key] = self.backend.alloc_device(max(nbytes_act, 16))
                self._gen[i] += 1  # handles to the old buffer are stale
        for key in ("x", "out"):
            pin = self._pinned.get(key)
            if pin is None or pin.nbytes < nbytes_act:
                self._quiesce()
                self._wait(("_x_ev",))
                if pin is not None:
                    self.backend.free_pinned_host(pin)
                self._pinned[key] = self.backend.alloc_pinned_host(max(nbytes_act, 16))
        self._reserved[bytes(desc)] = tokens

    def bind(self, layout: MoeLayerLayout, base: int, stream: Any) -> _lib.MxMoeWeights:
        """Weights of the layer buffer at ``base``; its expert pointer table is uploaded on
        ``stream`` the first time this layout is bound at this address."""
        self._last_stream = stream
        key = (id(layout), int(base))
        hit = self._tables.get(key)
        if hit is not None and hit[0] is layout:
            return hit[2]
        if len(self._tables) >= self.MAX_TABLES:
            self._quiesce()
            self._wait(("_table_ev",))
            for _, dev, _ in self._tables.values():
                self.backend.free_device(dev)
            self._tables.clear()
        nbytes = ctypes.sizeof(_lib.MxExpertPtrs) * (layout.n_experts + 1)
        pin = self._pinned.get("table")
        if pin is None or pin.nbytes < nbytes:
            self._wait(("_table_ev",))
            if pin is not None:
                self.backend.free_pinned_host(pin)
            pin = self._pinned["table"] = self.backend.alloc_pinned_host(max(nbytes, 4096))
        dev = self.backend.alloc_device(nbytes)
        table = layout.expert_table(base)
        # The previous upload may still be reading the pinned staging copy.
        self._wait(("_table_ev",))
        addr = ctypes.addressof(ctypes.c_char.from_buffer(pin.view))
        ctypes.memmove(addr, table, nbytes)
        self.backend.copy_h2d_ptr_async(dev.handle, addr, nbytes, stream)
        self._table_ev = self.backend.record_event(stream)
        w = layout.weights(base, dev.handle)
        self._tables[key] = (layout, dev, w)
        return w

    def _wait(self, names: tuple[str, ...]) -> None:
        for name in names:
            ev = getattr(self, name)
            if ev is not None:
                sync = getattr(self.backend, "event_synchronize", None)
                if sync is not None:
                    sync(ev)
                self.backend.destroy_event(ev)
                setattr(self, name, None)

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

    def _stage_input(self, desc: _lib.MxMoeDesc, x: Any, stream: Any,
                     pre: Callable[[int, int], None] | None,
                     fence: bool = False) -> tuple[int, int, int | None]:
        """Put the activations on the device; returns (tokens, device address, slot of that
        buffer or None for a caller-owned one).  NumPy goes up through pinned staging.  A
        ``DeviceActivations`` is read in place, or, when ``pre`` rewrites it, first copied
        into the input buffer so the caller's rows stay intact.  ``fence``: the call will not
        synchronise ``stream``, so the upload's end is recorded before the staging copy is
        written again."""
        self._last_stream = stream
        if isinstance(x, DeviceActivations):
            x.check()
            T, H = x.shape
            if H != desc.hidden:
                raise ValueError(f"activations must be [T, {desc.hidden}], got {x.shape}")
            self.reserve(desc, max(T, 1))
            if T and x.stream is not None and x.stream != stream:
                # produced on another stream: order this stream after it
                ev = self.backend.record_event(x.stream)
                self.backend.wait_event(stream, ev)
                self.backend.destroy_event(ev)
            if pre is None:
                return T, x.ptr, self._slot_of(x)
            if T:
                _lib.check(self.lib.mx_memcpy_d2d_async(self._io["x"].handle, x.ptr, x.nbytes,
                                                        stream), "hipMemcpyAsync")
                pre(self._io["x"].handle, T)
            return T, self._io["x"].handle, 0
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != desc.hidden:
            raise ValueError(f"activations must be [T, {desc.hidden}], got {x.shape}")
        T = x.shape[0]
        self.reserve(desc, max(T, 1))
        if T:
            px = self._pinned["x"]
            self._wait(("_x_ev",))  # the previous upload may still read the staging copy
            np.frombuffer(px.view, dtype=np.uint8, count=x.nbytes)[:] = x.view(np.uint8).ravel()
            self.backend.copy_h2d_ptr_async(self._io["x"].handle,
                                            ctypes.addressof(ctypes.c_char.from_buffer(px.view)),
                                            x.nbytes, stream)
            if fence:
                self._x_ev = self.backend.record_event(stream)
            if pre is not None:
                pre(self._io["x"].handle, T)
        return T, self._io["x"].handle, 0

    def _slot_of(self, x: DeviceActivations) -> int | None:
        return x._slot if x._owner is self else None

    def _pick_out(self, in_slot: int | None) -> int:
        slot = self._next_out
        if slot == in_slot:
            slot = 3 - slot
        self._next_out = 3 - slot
        return slot

    def _finish(self, desc: _lib.MxMoeDesc, T: int, slot: int, stream: Any,
                keep_on_device: bool) -> Any:
        out_buf = self._io[self._SLOTS[slot]]
        if keep_on_device:
            return DeviceActivations(self, slot, self._gen[slot], out_buf.handle, T,
                                     desc.hidden, stream)
        if T == 0:
            return np.zeros((0, desc.hidden), np.float32)
        nb = T * desc.hidden * 4
        po = self._pinned["out"]
        addr_o = ctypes.addressof(ctypes.c_char.from_buffer(po.view))
        self.backend.copy_d2h_ptr_async(addr_o, out_buf.handle, nb, stream)
        self.backend.synchronize_stream(stream)
        return np.frombuffer(po.view, dtype=np.float32, count=T * desc.hidden).reshape(T, -1).copy()

    def forward_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, x: Any,
                      stream: Any, pre: Callable[[int, int], None] | None = None,
                      keep_on_device: bool = False) -> Any:
        """MoE block of ``x`` (host fp32 [T, H] or ``DeviceActivations``).  Returns host
        fp32 [T, H] (synchronises ``stream``) or, with ``keep_on_device``, a
        ``DeviceActivations`` without waiting for the device.  ``pre(x_dev, T)``, when
        given, runs on ``stream`` on the device copy of x, rewriting it in place (for
        example the layer's attention block) before the MoE block reads it."""
        T, x_ptr, in_slot = self._stage_input(desc, x, stream, pre, fence=keep_on_device)
        slot = self._pick_out(in_slot)
        self._gen[slot] += 1  # handles to the previous contents of this buffer are stale
        if T:
            self.forward_device(desc, weights, x_ptr, self._io[self._SLOTS[slot]].handle, T,
                                stream)
        return self._finish(desc, T, slot, stream, keep_on_device)

    # -- split forward (router part, then the expert part after the experts are copied) --
    def route_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, x: Any,
                    stream: Any, pre: Callable[[int, int], None] | None = None) -> list[int]:
        """Stage x (then ``pre``) as ``forward_numpy`` does and run stages 0..3 (RMSNorm,
        router, top-k, dispatch); returns the routed experts the batch uses, ascending
        (synchronises ``stream``)."""
        T, x_ptr, in_slot = self._stage_input(desc, x, stream, pre)
        slot = self._pick_out(in_slot)
        self._gen[slot] += 1
        self._split = (T, slot, x_ptr)
        if T == 0:
            return []
        self._stages(desc, weights, T, x_ptr, slot, 0, _lib.MX_STAGE_ROUTE_END, stream)
        v = self.views(desc, T)
        ng = int(read_device(self.backend, v.n_groups, np.int32, 1, stream)[0])
        ge = read_device(self.backend, v.g_expert, np.int32, ng, stream)
        return sorted(int(e) for e in ge if e < desc.n_experts)

    def finish_numpy(self, desc: _lib.MxMoeDesc, weights: _lib.MxMoeWeights, stream: Any,
                     keep_on_device: bool = False) -> Any:
        """Stages 4..6 for the batch of the last ``route_numpy``; returns as
        ``forward_numpy`` does."""
        T, slot, x_ptr = self._split
        if T:
            self._stages(desc, weights, T, x_ptr, slot, _lib.MX_STAGE_ROUTE_END,
                         _lib.MX_N_STAGES, stream)
        return self._finish(desc, T, slot, stream, keep_on_device)

    def _stages(self, desc, weights, T: int, x_ptr: int, slot: int, begin: int, end: int,
                stream: Any) -> None:
        ws = self._ws
        _lib.check(self.lib.mx_moe_forward_stages(ctypes.byref(desc), ctypes.byref(weights),
                                                  x_ptr, self._io[self._SLOTS[slot]].handle,
                                                  T, ws.handle, ws.nbytes, begin, end, stream),
                   "mx_moe_forward_stages")

    # -- inspection --
    def views(self, desc: _lib.MxMoeDesc, tokens: int) -> _lib.MxMoeViews:
        v = _lib.MxMoeViews()
        _lib.check(self.lib.mx_moe_views(ctypes.byref(desc), tokens, self._ws.handle,
                                         ctypes.byref(v)), "mx_moe_views")
        return v

    def close(self) -> None:
        self._quiesce()
        self._wait(("_table_ev", "_x_ev"))
        bufs = [self._ws, *self._io.values(), *(dev for _, dev, _ in self._tables.values())]
        for buf in bufs:
            if buf is not None:
                self.backend.free_device(buf)
        for pin in self._pinned.values():
            self.backend.free_pinned_host(pin)
        self._ws = None
        self._tables.clear()
        self._io.clear()
        self._pinned.clear()
        self._reserved.clear()
        self._closed = True


def read_device(backend: MI355XBackend, ptr: int, dtype: Any, count: int, stream: Any = None) -> np.ndarray:
    """Synchronous copy of ``count`` elements at a device address into a new array."""
    out = np.empty(count, dtype=dtype)
    if count:
        backend.copy_d2h_ptr_async(out.ctypes.data, ptr, out.nbytes, stream)
        backend.synchronize_stream(stream)
    return out
