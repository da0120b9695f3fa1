"""Layer executors whose MoE step runs on the MI355X.

Drop-ins for ``GLM4MoeExecutor`` (offload_runtime/executors/glm4_moe.py:63-249) and
``Qwen3NextExecutor`` (offload_runtime/executors/qwen3_next.py:102-342) behind the
``LayerExecutor.run_layer`` contract (offload_runtime/runtime.py:15-26).  Only the MoE
step ``_moe_mlp_block`` is replaced: it consumes the layer's ``DeviceBuffer`` in place
(no read-back of expert weights) through a device pointer table built from
``layer.metadata["tensors"]`` offsets.

Attention is not part of this package.  ``run_layer`` runs layers that hold only the MoE
block tensors directly; for full transformer layers pass ``attention=callable``, which
receives ``(x, layer, device_weights, backend, stream)`` and returns the post-attention
activations.  ``host_attention(fn)`` builds one from a host function ``fn(x, tensors)`` (for
example the reference executor's own ``_attention_block``): it copies back only the
layer's non-MLP tensors (``read_layer_tensors``) where the reference reads back the whole
layer (glm4_moe.py:96-97, _common.py:20-34).

GLM4-MoE layers whose ``metadata["is_moe"]`` is false or absent (the reference's default,
glm4_moe.py:102: the ``first_k_dense_replace`` layers) run a dense MLP, which is not part
of the MoE path either: pass ``dense=callable`` with the same signature as ``attention``;
``host_dense(fn)`` runs ``fn(x, tensors)`` on the host over the layer's
``post_attention_layernorm`` and ``mlp.{gate,up,down}_proj`` tensors (for example the
reference's ``_dense_mlp_block``, glm4_moe.py:166-172).

Before ``run_layer`` returns, the compute stream is synchronised: the runtime frees or
re-pools ``device_weights`` right after the call (runtime.py:180).  Under a runtime that
fences buffer reuse with events (``stream_ordered``, set by ``moe_mi355x.OffloadRuntime``)
and with ``device_activations=True``, ``run_layer`` returns without waiting: the output
stays on the device as ``DeviceActivations`` and the next layer reads it in place.
"""
from __future__ import annotations

from typing import Any, Callable

import numpy as np

from . import _lib
from .layout import NORM, MoeLayerLayout
from .full_attn import FullAttnLayout, FullAttnRunner, has_full_attn
from .linear_attn import LinearAttnLayout, LinearAttnRunner, has_linear_attn
from .activations import DeviceActivations
from .moe import MoeConfig, MoeRunner
from .types import DeviceBuffer, HostBuffer, LayerSpec

AttentionFn = Callable[[np.ndarray, LayerSpec, DeviceBuffer, Any, Any], np.ndarray]


def _rms_norm_np(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    return w * (x / rms)


def _merge_ranges(ranges: list[tuple[int, int]], gap: int) -> list[tuple[int, int]]:
    """Sorted, merged byte ranges; ranges less than ``gap`` bytes apart are joined."""
    out: list[tuple[int, int]] = []
    for a, b in sorted(ranges):
        if out and a - out[-1][1] < gap:
            out[-1] = (out[-1][0], max(out[-1][1], b))
        else:
            out.append((a, b))
    return out


def read_layer_tensors(layer: LayerSpec, device_weights: DeviceBuffer, backend: Any,
                       stream: Any, keep: Callable[[str], bool] | None = None,
                       gap: int = 1 << 16) -> dict[str, np.ndarray]:
    """Copy the tensors ``keep`` selects (by default every tensor outside the MoE block:
    the attention weights and ``input_layernorm``) back to the host and return them by name.

    Only the selected byte ranges travel (neighbours closer than ``gap`` bytes share one
    copy); backends without pointer copies read the whole layer back, as
    _common.py:20-34 does.  The stream is synchronised before returning.
    """
    keep = keep or (lambda n: not n.startswith("mlp.") and n != NORM)
    metas = [m for m in layer.metadata["tensors"] if keep(m["name"])]
    out: dict[str, np.ndarray] = {}
    if not metas:
        return out

    def view(chunk: np.ndarray, base: int, m: dict[str, Any]) -> np.ndarray:
        dt = np.dtype(m["dtype"])
        a = m["offset"] - base
        return chunk[a:a + m["nbytes"]].view(dt).reshape(m["shape"])

    if not hasattr(backend, "copy_d2h_ptr_async"):
        buf = np.empty(device_weights.nbytes, np.uint8)
        backend.copy_d2h_async(HostBuffer(view=memoryview(buf)), device_weights, stream)
        backend.synchronize_stream(stream)
        return {m["name"]: view(buf, 0, m) for m in metas}
    spans = _merge_ranges([(m["offset"], m["offset"] + m["nbytes"]) for m in metas], gap)
    chunks = []
    for a, b in spans:
        chunk = np.empty(b - a, np.uint8)
        backend.copy_d2h_ptr_async(int(chunk.ctypes.data), int(device_weights.handle) + a,
                                   b - a, stream)
        chunks.append((a, b, chunk))
    backend.synchronize_stream(stream)
    for m in metas:
        a, _, chunk = next(c for c in chunks if c[0] <= m["offset"] < c[1] or
                           (m["nbytes"] == 0 and c[0] <= m["offset"] <= c[1]))
        out[m["name"]] = view(chunk, a, m)
    return out


def host_attention(fn: Callable[[np.ndarray, dict[str, np.ndarray]], np.ndarray],
                   keep: Callable[[str], bool] | None = None) -> AttentionFn:
    """An ``attention=`` hook that runs ``fn(x, tensors)`` on the host over the layer's
    non-MLP tensors, copied back by ``read_layer_tensors``."""

    def run(x: np.ndarray, layer: LayerSpec, device_weights: DeviceBuffer, backend: Any,
            stream: Any) -> np.ndarray:
        t = read_layer_tensors(layer, device_weights, backend, stream, keep)
        return np.asarray(fn(x, t), dtype=np.float32)

    return run


def _dense_tensor(name: str) -> bool:
    return name == NORM or name in {f"mlp.{p}.weight" for p in ("gate_proj", "up_proj",
                                                                 "down_proj")}


def host_dense(fn: Callable[[np.ndarray, dict[str, np.ndarray]], np.ndarray]) -> AttentionFn:
    """A ``dense=`` hook that runs ``fn(x, tensors)`` on the host over the dense MLP tensors
    of the layer (``post_attention_layernorm.weight``, ``mlp.{gate,up,down}_proj.weight``),
    copied back by ``read_layer_tensors``."""
    return host_attention(fn, keep=_dense_tensor)


class _MoeExecutorBase:
    _router_default: int = _lib.MX_ROUTER_REF_SOFTMAX_BIAS

    def __init__(self, config: dict[str, Any], *, router_mode: int | str | None = None,
                 attention: AttentionFn | None = None, dense: AttentionFn | None = None,
                 max_tokens: int = 32, device_activations: bool = False) -> None:
        self.hidden_size = int(config["hidden_size"])
        self.router_mode = router_mode if router_mode is not None else self._router_default
        self.attention = attention
        self.dense = dense
        self.max_tokens = max_tokens
        # run_layer returns DeviceActivations (the next layer reads them in place) instead
        # of NumPy; inputs may be either in both modes.
        self.device_activations = bool(device_activations)
        # Set by a runtime that records an event on the compute stream after run_layer and
        # fences every reuse or free of the layer buffer on it (moe_mi355x.OffloadRuntime
        # does).  The reference runtime frees the buffer right after run_layer returns
        # (runtime.py:180), so by default run_layer waits for its device work.
        self.stream_ordered = False
        self._runner: MoeRunner | None = None
        self._layouts: dict[int, tuple[list, MoeLayerLayout]] = {}
        self._la_runner: LinearAttnRunner | None = None
        self._la_layouts: dict[int, tuple[list, LinearAttnLayout]] = {}
        self._fa_runner: FullAttnRunner | None = None
        self._fa_layouts: dict[int, tuple[list, FullAttnLayout]] = {}
        self._facts: dict[tuple[int, str], tuple[list, Any]] = {}

    # values supplied by subclasses
    top_k: int
    norm_topk_prob: bool
    routed_scaling: float
    rms_norm_eps: float

    def _desc(self, layer: LayerSpec, layout: MoeLayerLayout) -> Any:
        """The block descriptor of a layer, built once per (layer, tensor list, layout
        flag, router settings)."""
        key = (layer.layer_id, "desc")
        meta = layer.metadata["tensors"]
        stamp = (layer.metadata.get("weight_layout"), self.router_mode, self.top_k,
                 self.norm_topk_prob, self.routed_scaling, self.rms_norm_eps)
        hit = self._facts.get(key)
        if hit is not None and hit[0] is meta and hit[1][0] == stamp:
            return hit[1][1]
        desc = self.moe_config(layout, layer).desc()
        self._facts[key] = (meta, (stamp, desc))
        return desc

    def _cached(self, layer: LayerSpec, key: str, fn: Callable[[LayerSpec], bool]) -> bool:
        """A per-layer fact derived from its tensor list (a scan of every tensor name),
        computed once per (layer, tensor list)."""
        meta = layer.metadata["tensors"]
        hit = self._facts.get((layer.layer_id, key))
        if hit is not None and hit[0] is meta:
            return hit[1]
        v = bool(fn(layer))
        self._facts[(layer.layer_id, key)] = (meta, v)
        return v

    def _layout(self, layer: LayerSpec) -> MoeLayerLayout:
        meta = layer.metadata["tensors"]
        hit = self._layouts.get(layer.layer_id)
        if hit is not None and hit[0] is meta:
            return hit[1]
        lay = MoeLayerLayout.from_meta(meta)
        if lay.hidden != self.hidden_size:
            raise ValueError(f"layer hidden size {lay.hidden} != config {self.hidden_size}")
        self._layouts[layer.layer_id] = (meta, lay)
        return lay

    def moe_config(self, layout: MoeLayerLayout, layer: LayerSpec | None = None) -> MoeConfig:
        """Block configuration; a layer whose expert matrices were re-laid in the
        fragment layout on the device says so with ``metadata["weight_layout"] = "frag16"``."""
        wl = _lib.MX_LAYOUT_ROWS
        if layer is not None and layer.metadata.get("weight_layout", "rows") == "frag16":
            wl = _lib.MX_LAYOUT_FRAG16
        return MoeConfig.from_layout(layout, top_k=self.top_k, router_mode=self.router_mode,
                                     norm_topk_prob=self.norm_topk_prob,
                                     routed_scaling=self.routed_scaling, eps=self.rms_norm_eps,
                                     weight_layout=wl)

    def moe_block(self, layer: LayerSpec, x: np.ndarray, device_weights: DeviceBuffer,
                  backend: Any, stream: Any, pre: Callable[[int, int], None] | None = None
                  ) -> np.ndarray:
        """x + MoE(rms_norm(x)) on the device (the reference ``_moe_mlp_block``); ``pre``
        rewrites the uploaded activations on the device first (the attention block)."""
        if device_weights.backend != "rocm":
            raise RuntimeError("the MoE step needs the MI355X backend; got "
                               f"{device_weights.backend!r} device buffers")
        if device_weights.nbytes < layer.nbytes:
            raise RuntimeError(f"Layer {layer.layer_id}: device buffer size "
                               f"{device_weights.nbytes} < expected {layer.nbytes}")
        layout = self._layout(layer)
        desc = self._desc(layer, layout)
        if self._runner is None:
            self._runner = MoeRunner(backend)
        T = len(x)
        self._runner.reserve(desc, max(T, self.max_tokens, 1))
        weights = self._runner.bind(layout, int(device_weights.handle), stream)
        out = self._runner.forward_numpy(desc, weights, x, stream, pre=pre,
                                         keep_on_device=self.device_activations)
        return self._fence(out, backend, stream)

    def _fence(self, out: Any, backend: Any, stream: Any) -> Any:
        """Device output under a caller that does not fence buffer reuse: wait for the
        device work before the layer buffer can be freed (NumPy output already waited)."""
        if isinstance(out, DeviceActivations) and not self.stream_ordered:
            backend.synchronize_stream(stream)
        return out

    def moe_block_granular(self, layer: LayerSpec, x: np.ndarray, device_weights: DeviceBuffer,
                           backend: Any, stream: Any, fetch: Callable[[list[int]], None],
                           pre: Callable[[int, int], None] | None = None) -> np.ndarray:
        """The MoE step when only the layer's non-expert bytes are on the device yet: route
        on the device, ``fetch(expert_ids)`` (the caller copies those routed experts into
        ``device_weights`` and makes ``stream`` wait for the copies), then the experts."""
        if device_weights.backend != "rocm":
            raise RuntimeError("the MoE step needs the MI355X backend; got "
                               f"{device_weights.backend!r} device buffers")
        if device_weights.nbytes < layer.nbytes:
            raise RuntimeError(f"Layer {layer.layer_id}: device buffer size "
                               f"{device_weights.nbytes} < expected {layer.nbytes}")
        layout = self._layout(layer)
        desc = self._desc(layer, layout)
        if self._runner is None:
            self._runner = MoeRunner(backend)
        T = len(x)
        self._runner.reserve(desc, max(T, self.max_tokens, 1))
        weights = self._runner.bind(layout, int(device_weights.handle), stream)
        active = self._runner.route_numpy(desc, weights, x, stream, pre=pre)
        fetch(active)
        out = self._runner.finish_numpy(desc, weights, stream,
                                        keep_on_device=self.device_activations)
        return self._fence(out, backend, stream)

    def expert_ranges(self, layer: LayerSpec) -> tuple[list[tuple[int, int]], list[tuple[int, int]]]:
        """(core byte ranges, per-routed-expert byte ranges) of a packed MoE layer."""
        lay = self._layout(layer)
        return lay.core_ranges(layer.nbytes), lay.routed_expert_ranges()

    def _attention(self, layer: LayerSpec, x: np.ndarray, device_weights: DeviceBuffer,
                   backend: Any, stream: Any) -> tuple[np.ndarray, Any]:
        """Run (host hook) or schedule (device block, returned as a ``pre`` hook) the
        layer's attention part."""
        if self.attention is not None:
            return self.attention(np.asarray(x, dtype=np.float32), layer, device_weights,
                                  backend, stream), None
        pre = self._device_attention(layer, device_weights, backend, stream)
        if pre is None and not self._cached(layer, "moe_only", self._moe_only):
            raise NotImplementedError(
                "layer holds attention tensors; pass attention=... to run them")
        return x, pre

    def _device_attention(self, layer: LayerSpec, device_weights: DeviceBuffer, backend: Any,
                          stream: Any) -> Callable[[int, int], None] | None:
        return None

    def run_layer_granular(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                           backend: Any, stream: Any, fetch: Callable[[list[int]], None]) -> Any:
        """``run_layer`` for a layer whose routed experts are copied on demand."""
        x, pre = self._attention(layer, self._as_input(activations), device_weights, backend,
                                 stream)
        return self.moe_block_granular(layer, x, device_weights, backend, stream, fetch, pre=pre)

    def is_moe_layer(self, layer: LayerSpec) -> bool:
        """Whether the layer's MLP is the MoE block (else a dense MLP)."""
        return True

    @staticmethod
    def _as_input(activations: Any) -> Any:
        if isinstance(activations, DeviceActivations):
            return activations
        return np.asarray(activations, dtype=np.float32)

    def run_layer(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                  backend: Any, stream: Any) -> Any:
        """The reference contract (runtime.py:15-26): the layer's output activations.
        ``activations`` may be NumPy or ``DeviceActivations``; the result is NumPy, or
        ``DeviceActivations`` for an executor built with ``device_activations=True``."""
        x, pre = self._attention(layer, self._as_input(activations), device_weights, backend,
                                 stream)
        if not self.is_moe_layer(layer):
            if self.dense is None:
                raise NotImplementedError(
                    f"layer {layer.layer_id} is a dense MLP layer (metadata is_moe false); "
                    "pass dense=... (for example host_dense(fn)) to run it")
            if pre is not None:
                raise NotImplementedError("a dense MLP after a device attention block")
            return np.asarray(self.dense(np.asarray(x, dtype=np.float32), layer,
                                         device_weights, backend, stream), dtype=np.float32)
        return self.moe_block(layer, x, device_weights, backend, stream, pre=pre)

    @staticmethod
    def _moe_only(layer: LayerSpec) -> bool:
        return all(m["name"] == NORM or m["name"].startswith("mlp.")
                   for m in layer.metadata["tensors"])

    # -- non-layer helpers (glm4_moe.py:244-249, qwen3_next.py:337-342) --
    def embed(self, token_ids: list[int], embed_weights: Any) -> Any:
        out = embed_weights[token_ids]
        return out if out.dtype == np.float32 else out.astype(np.float32)

    def lm_head(self, hidden: Any, norm_w: Any, head_w: Any) -> Any:
        return _rms_norm_np(hidden, norm_w, self.rms_norm_eps) @ head_w.T

    def close(self) -> None:
        if self._runner is not None:
            self._runner.close()
            self._runner = None
        if self._la_runner is not None:
            self._la_runner.close()
            self._la_runner = None
        if self._fa_runner is not None:
            self._fa_runner.close()
            self._fa_runner = None


class GLM4MoeExecutor(_MoeExecutorBase):
    """GLM4-MoE (Glm4MoeForCausalLM).  Default router mode reproduces the reference
    (softmax over logits + correction bias); ``router_mode="sigmoid_select_bias"``
    gives the checkpoint semantics (sigmoid scores, bias for selection only)."""

    _router_default = _lib.MX_ROUTER_REF_SOFTMAX_BIAS

    def __init__(self, config: dict[str, Any], **kw: Any) -> None:
        super().__init__(config, **kw)
        self.rms_norm_eps = float(config.get("rms_norm_eps", 1e-5))
        self.top_k = int(config.get("num_experts_per_tok", 8))
        self.n_routed_experts = int(config.get("n_routed_experts", 160))
        self.routed_scaling = float(config.get("routed_scaling_factor", 2.5))
        self.norm_topk_prob = bool(config.get("norm_topk_prob", True))
        self.num_experts_per_tok = self.top_k
        self.routed_scaling_factor = self.routed_scaling

    def is_moe_layer(self, layer: LayerSpec) -> bool:
        # glm4_moe.py:102: a layer without the flag is a dense (first_k_dense_replace) layer.
        return bool(layer.metadata.get("is_moe", False))


class Qwen3NextExecutor(_MoeExecutorBase):
    """Qwen3-Next (Qwen3NextForCausalLM): softmax router, renormalised top-k, no scaling,
    shared expert scaled by sigmoid(h . shared_expert_gate).

    Both attention kinds run on the device ahead of the MoE block, on the same uploaded
    activations: linear-attention layers (``metadata["attn_type"]`` "linear", the default as
    in qwen3_next.py:155) their Gated DeltaNet block, full-attention layers ("full") their
    gated softmax attention (qwen3_next.py:161-205)."""

    _router_default = _lib.MX_ROUTER_SOFTMAX

    def __init__(self, config: dict[str, Any], **kw: Any) -> None:
        super().__init__(config, **kw)
        self.rms_norm_eps = float(config.get("rms_norm_eps", 1e-6))
        # qwen3_next.py:120-125
        self.linear_num_key_heads = int(config.get("linear_num_key_heads", 16))
        self.linear_key_head_dim = int(config.get("linear_key_head_dim", 128))
        self.linear_num_value_heads = int(config.get("linear_num_value_heads", 32))
        self.linear_value_head_dim = int(config.get("linear_value_head_dim", 128))
        self.linear_conv_kernel_dim = int(config.get("linear_conv_kernel_dim", 4))
        # qwen3_next.py:109-118 (num_attention_heads is required there for full layers)
        heads = config.get("num_attention_heads")
        self.num_heads = int(heads) if heads is not None else None
        self.num_kv_heads = int(config.get("num_key_value_heads", heads or 1))
        self.head_dim = int(config.get("head_dim", self.hidden_size // (self.num_heads or 1)))
        self.partial_rotary_factor = float(config.get("partial_rotary_factor", 0.25))
        self.rotary_dim = int(self.head_dim * self.partial_rotary_factor)
        self.rope_theta = float(config.get("rope_theta", 5000000.0))
        self.num_experts = int(config.get("num_experts", config.get("n_routed_experts", 512)))
        self.top_k = int(config.get("num_experts_per_tok", 10))
        self.norm_topk_prob = bool(config.get("norm_topk_prob", True))
        self.routed_scaling = 1.0
        self.num_experts_per_tok = self.top_k

    def linear_attn_layout(self, layer: LayerSpec) -> LinearAttnLayout:
        meta = layer.metadata["tensors"]
        hit = self._la_layouts.get(layer.layer_id)
        if hit is not None and hit[0] is meta:
            return hit[1]
        if self.linear_num_key_heads != self.linear_num_value_heads:
            # qwen3_next.py:75-77 reshapes q/k [T, key heads * dk] with the value-head
            # count, which fails unless the counts agree.
            raise ValueError(
                f"linear attention needs linear_num_key_heads == linear_num_value_heads "
                f"(got {self.linear_num_key_heads} and {self.linear_num_value_heads})")
        lay = LinearAttnLayout.from_meta(meta)
        want = (self.hidden_size, self.linear_num_value_heads, self.linear_key_head_dim,
                self.linear_value_head_dim, self.linear_conv_kernel_dim)
        got = (lay.hidden, lay.n_heads, lay.head_dim_k, lay.head_dim_v, lay.conv_kernel)
        if got != want:
            raise ValueError(f"layer {layer.layer_id}: linear-attention tensors give "
                             f"(hidden, heads, dk, dv, conv) = {got}, config says {want}")
        self._la_layouts[layer.layer_id] = (meta, lay)
        return lay

    def full_attn_layout(self, layer: LayerSpec) -> FullAttnLayout:
        meta = layer.metadata["tensors"]
        hit = self._fa_layouts.get(layer.layer_id)
        if hit is not None and hit[0] is meta:
            return hit[1]
        if self.num_heads is None:
            raise ValueError("full-attention layers need num_attention_heads in the config")
        lay = FullAttnLayout.from_meta(meta, self.num_heads, self.num_kv_heads, self.head_dim,
                                       self.rotary_dim, self.rope_theta)
        self._fa_layouts[layer.layer_id] = (meta, lay)
        return lay

    def _device_attention(self, layer: LayerSpec, device_weights: DeviceBuffer, backend: Any,
                          stream: Any) -> Callable[[int, int], None] | None:
        kind = layer.metadata.get("attn_type", "linear")
        if kind == "full" and self._cached(layer, "full", lambda l: has_full_attn(
                l.metadata["tensors"])):
            return self._device_full_attention(layer, device_weights, backend, stream)
        if kind != "linear" or not self._cached(layer, "linear", lambda l: has_linear_attn(
                l.metadata["tensors"])):
            return None
        if device_weights.backend != "rocm":
            raise RuntimeError("the linear-attention block needs the MI355X backend; got "
                               f"{device_weights.backend!r} device buffers")
        lay = self.linear_attn_layout(layer)
        desc = lay.desc(self.rms_norm_eps)
        weights = lay.weights(int(device_weights.handle))
        if self._la_runner is None:
            self._la_runner = LinearAttnRunner(backend)
        runner = self._la_runner

        def pre(x_dev: int, tokens: int) -> None:
            runner.reserve(desc, max(tokens, self.max_tokens, 1), io=False)
            runner.forward_device(desc, weights, x_dev, x_dev, tokens, stream)

        return pre

    def _device_full_attention(self, layer: LayerSpec, device_weights: DeviceBuffer,
                               backend: Any, stream: Any) -> Callable[[int, int], None]:
        if device_weights.backend != "rocm":
            raise RuntimeError("the attention block needs the MI355X backend; got "
                               f"{device_weights.backend!r} device buffers")
        lay = self.full_attn_layout(layer)
        desc = lay.desc(self.rms_norm_eps)
        weights = lay.weights(int(device_weights.handle))
        if self._fa_runner is None:
            self._fa_runner = FullAttnRunner(backend)
        runner = self._fa_runner

        def pre(x_dev: int, tokens: int) -> None:
            runner.reserve(desc, max(tokens, self.max_tokens, 1), io=False)
            runner.forward_device(desc, weights, x_dev, x_dev, tokens, stream)

        return pre

    @staticmethod
    def _moe_only(layer: LayerSpec) -> bool:
        return all(m["name"] in (NORM, "input_layernorm.weight") or
                   m["name"].startswith(("mlp.", "linear_attn."))
                   for m in layer.metadata["tensors"]) and \
            layer.metadata.get("attn_type", "linear") == "linear"
