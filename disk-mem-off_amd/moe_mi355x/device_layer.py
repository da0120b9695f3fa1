"""A packed MoE layer resident in HBM plus the runner that executes it.

Two ways to populate the layer buffer:
  * ``DeviceMoeLayer.from_host``: pack host arrays (loader layout, ``align`` padding) and
    copy them in through pinned memory;
  * ``DeviceMoeLayer.synthetic``: lay the buffer out from the tensor specs and generate
    the expert weights directly on the device with ``mx_fill_normal`` (the same values
    ``synthetic.make_tensors`` produces on the host), quantising to per-row int8 on the
    device when asked.  This is how multi-GB benchmark layers are built without host
    round trips.
"""
from __future__ import annotations

import ctypes
from typing import Any

import numpy as np

from . import _lib, gen
from .backends import MI355XBackend
from .layout import MoeLayerLayout, frag16_to_rows, make_layer_spec, pack_tensors
from .moe import MoeConfig, MoeRunner, tile_experts
from .synthetic import MoeShape, stream_of, tensor_specs
from .types import DeviceBuffer, LayerSpec

_NP_DT = {"float32": np.float32, "float16": np.float16, "int8": np.int8}


def _upload(backend: MI355XBackend, dst: int, arr: np.ndarray, stream: Any) -> None:
    arr = np.ascontiguousarray(arr)
    if arr.nbytes == 0:
        return
    pin = backend.alloc_pinned_host(arr.nbytes)
    try:
        np.frombuffer(pin.view, dtype=np.uint8, count=arr.nbytes)[:] = arr.view(np.uint8).ravel()
        backend.copy_h2d_ptr_async(dst, ctypes.addressof(ctypes.c_char.from_buffer(pin.view)),
                                   arr.nbytes, stream)
        backend.synchronize_stream(stream)
    finally:
        backend.free_pinned_host(pin)


class DeviceMoeLayer:
    def __init__(self, backend: MI355XBackend, layer: LayerSpec, buf: DeviceBuffer,
                 stream: Any) -> None:
        self.backend = backend
        self.layer = layer
        self.buf = buf
        self.stream = stream
        self.layout = MoeLayerLayout.from_meta(layer.metadata["tensors"])
        self.runner = MoeRunner(backend)
        self._weights = None
        self.weight_layout = _lib.MX_LAYOUT_ROWS

    def tile(self) -> "DeviceMoeLayer":
        """Re-lay the expert weights in place into MX_LAYOUT_FRAG16 (one device pass); the
        configs made afterwards carry the layout."""
        if self.weight_layout != _lib.MX_LAYOUT_FRAG16:
            tile_experts(self.backend, self.layout, self.buf.handle, self.stream)
            self.weight_layout = _lib.MX_LAYOUT_FRAG16
        return self

    # -- construction --
    @classmethod
    def from_host(cls, backend: MI355XBackend, tensors: dict[str, np.ndarray], stream: Any,
                  align: int = 256, layer_id: int = 0) -> "DeviceMoeLayer":
        raw, meta = pack_tensors(tensors, align=align)
        layer = make_layer_spec(layer_id, meta, len(raw))
        buf = backend.alloc_device(len(raw))
        _upload(backend, buf.handle, np.frombuffer(raw, dtype=np.uint8), stream)
        return cls(backend, layer, buf, stream)

    @staticmethod
    def synthetic_meta(shape: MoeShape, weight_dtype: str = "float16",
                       param_dtype: str = "float32", align: int = 256) -> list[dict[str, Any]]:
        entries = []
        for name, shp, kind, std in tensor_specs(shape):
            is_expert = name.startswith(("mlp.experts.", "mlp.shared_experts.",
                                         "mlp.shared_expert."))
            dt = weight_dtype if is_expert else param_dtype
            entries.append((name, list(shp), dt))
            if is_expert and dt == "int8":
                entries.append((name + "_scale", [shp[0]], "float16"))
        entries.sort(key=lambda e: e[0])
        meta, off = [], 0
        for name, shp, dt in entries:
            off = (off + align - 1) // align * align
            nbytes = int(np.prod(shp)) * np.dtype(dt).itemsize
            meta.append({"name": name, "shape": shp, "dtype": dt, "offset": off, "nbytes": nbytes})
            off += nbytes
        return meta

    @classmethod
    def synthetic(cls, backend: MI355XBackend, shape: MoeShape, seed: int, stream: Any,
                  weight_dtype: str = "float16", param_dtype: str = "float32",
                  bias: np.ndarray | None = None, norm_noise: float = 0.0,
                  layer_id: int = 0) -> "DeviceMoeLayer":
        """Generate the layer on the device.  ``bias`` overrides the correction bias."""
        meta = cls.synthetic_meta(shape, weight_dtype, param_dtype)
        total = meta[-1]["offset"] + meta[-1]["nbytes"]
        layer = make_layer_spec(layer_id, meta, total)
        buf = backend.alloc_device(total)
        lib = _lib.load()
        by_name = {m["name"]: m for m in meta}
        specs = {n: (tuple(s), k, std) for n, s, k, std in tensor_specs(shape)}
        tmp: DeviceBuffer | None = None
        try:
            for name, (shp, kind, std) in specs.items():
                m = by_name[name]
                dst = buf.handle + m["offset"]
                n = int(np.prod(shp))
                if kind == "norm":
                    v = np.ones(shp, np.float32)
                    if norm_noise:
                        v = v + gen.normal(seed, stream_of(name), shp, std=norm_noise)
                    _upload(backend, dst, v.astype(_NP_DT[m["dtype"]]), stream)
                elif kind == "bias" and bias is not None:
                    _upload(backend, dst, np.asarray(bias, np.float32).astype(_NP_DT[m["dtype"]]),
                            stream)
                elif m["dtype"] in ("float32", "float16"):
                    code = _lib.MX_DT_F32 if m["dtype"] == "float32" else _lib.MX_DT_F16
                    _lib.check(lib.mx_fill_normal(dst, code, n, seed, stream_of(name), 0, std,
                                                  stream), "mx_fill_normal")
                else:  # int8 expert weight: fp32 draw, then per-row quantisation
                    if tmp is None or tmp.nbytes < n * 4:
                        if tmp is not None:
                            backend.synchronize_stream(stream)
                            backend.free_device(tmp)
                        tmp = backend.alloc_device(n * 4)
                    _lib.check(lib.mx_fill_normal(tmp.handle, _lib.MX_DT_F32, n, seed,
                                                  stream_of(name), 0, std, stream),
                               "mx_fill_normal")
                    sc = by_name[name + "_scale"]
                    _lib.check(lib.mx_quantize_rows_i8(tmp.handle, _lib.MX_DT_F32, shp[0], shp[1],
                                                       dst, buf.handle + sc["offset"], stream),
                               "mx_quantize_rows_i8")
            backend.synchronize_stream(stream)
        finally:
            if tmp is not None:
                backend.synchronize_stream(stream)
                backend.free_device(tmp)
        return cls(backend, layer, buf, stream)

    # -- running --
    def config(self, *, top_k: int, router_mode: int | str, routed_scaling: float, eps: float,
               norm_topk_prob: bool = True) -> MoeConfig:
        return MoeConfig.from_layout(self.layout, top_k=top_k, router_mode=router_mode,
                                     norm_topk_prob=norm_topk_prob, routed_scaling=routed_scaling,
                                     eps=eps, weight_layout=self.weight_layout)

    def prepare(self, cfg: MoeConfig, max_tokens: int) -> _lib.MxMoeWeights:
        self.runner.reserve(cfg.desc(), max_tokens)
        self._weights = self.runner.bind(self.layout, self.buf.handle, self.stream)
        self.backend.synchronize_stream(self.stream)
        return self._weights

    def forward_numpy(self, cfg: MoeConfig, x: np.ndarray) -> np.ndarray:
        w = self.prepare(cfg, max(1, x.shape[0]))
        return self.runner.forward_numpy(cfg.desc(), w, x, self.stream)

    def read(self, name: str) -> np.ndarray:
        """Copy one tensor of the layer back to the host."""
        m = self.layout.entries[name]
        out = np.empty(m["shape"], dtype=_NP_DT[m["dtype"]])
        self.backend.copy_d2h_ptr_async(out.ctypes.data, self.buf.handle + m["offset"],
                                        out.nbytes, self.stream)
        self.backend.synchronize_stream(self.stream)
        if self.weight_layout == _lib.MX_LAYOUT_FRAG16 and out.ndim == 2 and \
                any(o == m["offset"] for o, _, _ in self.layout.expert_matrices()):
            out = frag16_to_rows(out, out.shape[0], out.shape[1], out.dtype)
        return out

    def to_pinned(self) -> Any:
        """A copy of the whole layer buffer in a new pinned host buffer (``HostBuffer``; the
        caller frees it with ``free_pinned_host``): a layer as the offload runtime streams
        it from host memory."""
        pin = self.backend.alloc_pinned_host(self.layer.nbytes)
        try:
            self.backend.copy_d2h_ptr_async(ctypes.addressof(ctypes.c_char.from_buffer(pin.view)),
                                            self.buf.handle, self.layer.nbytes, self.stream)
            self.backend.synchronize_stream(self.stream)
        except BaseException:
            self.backend.free_pinned_host(pin)
            raise
        return pin

    def write(self, offset: int, arr: np.ndarray) -> None:
        """Copy a host array into the layer buffer at byte ``offset`` (synchronous)."""
        arr = np.ascontiguousarray(arr)
        if offset < 0 or offset + arr.nbytes > self.buf.nbytes:
            raise ValueError(f"write of {arr.nbytes} bytes at {offset} outside the layer "
                             f"buffer ({self.buf.nbytes} bytes)")
        _upload(self.backend, self.buf.handle + offset, arr, self.stream)

    def read_tensors(self, names: list[str]) -> dict[str, np.ndarray]:
        out = {}
        for n in names:
            out[n] = self.read(n)
            if n + "_scale" in self.layout.entries:
                out[n + "_scale"] = self.read(n + "_scale")
        return out

    def close(self) -> None:
        self.backend.synchronize_stream(self.stream)
        self.runner.close()
        self.backend.free_device(self.buf)
