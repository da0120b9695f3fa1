"""Layer executors whose MoE step runs on the MI355X.

Drop-ins for ``GLM4MoeExecutor`` (offload_runtime/executors/glm4_moe.py:63-249) and
``Qwen3NextExecutor`` (offload_runtime/executors/qwen3_next.py:102-342) behind the
``LayerExecutor.run_layer`` contract (offload_runtime/runtime.py:15-26).  Only the MoE
step ``_moe_mlp_block`` is replaced: it consumes the layer's ``DeviceBuffer`` in place
(no read-back of expert weights) through a device pointer table built from
``layer.metadata["tensors"]`` offsets.

Attention is not part of this package.  ``run_layer`` runs layers that hold only the MoE
block tensors directly; for full transformer layers pass ``attention=callable`` (for
example the reference executor's own ``_attention_block`` over read-back attention
tensors), which receives ``(x, layer, device_weights, backend, stream)`` and returns the
post-attention activations.

Before ``run_layer`` returns, the compute stream is synchronised: the runtime frees or
re-pools ``device_weights`` right after the call (runtime.py:180).
"""
from __future__ import annotations

from typing import Any, Callable

import numpy as np

from . import _lib
from .layout import NORM, MoeLayerLayout
from .moe import MoeConfig, MoeRunner
from .types import DeviceBuffer, LayerSpec

AttentionFn = Callable[[np.ndarray, LayerSpec, DeviceBuffer, Any, Any], np.ndarray]


def _rms_norm_np(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    return w * (x / rms)


class _MoeExecutorBase:
    _router_default: int = _lib.MX_ROUTER_REF_SOFTMAX_BIAS

    def __init__(self, config: dict[str, Any], *, router_mode: int | str | None = None,
                 attention: AttentionFn | None = None, max_tokens: int = 32) -> None:
        self.hidden_size = int(config["hidden_size"])
        self.router_mode = router_mode if router_mode is not None else self._router_default
        self.attention = attention
        self.max_tokens = max_tokens
        self._runner: MoeRunner | None = None
        self._layouts: dict[int, tuple[list, MoeLayerLayout]] = {}

    # values supplied by subclasses
    top_k: int
    norm_topk_prob: bool
    routed_scaling: float
    rms_norm_eps: float

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

    def moe_config(self, layout: MoeLayerLayout) -> MoeConfig:
        return MoeConfig.from_layout(layout, top_k=self.top_k, router_mode=self.router_mode,
                                     norm_topk_prob=self.norm_topk_prob,
                                     routed_scaling=self.routed_scaling, eps=self.rms_norm_eps)

    def moe_block(self, layer: LayerSpec, x: np.ndarray, device_weights: DeviceBuffer,
                  backend: Any, stream: Any) -> np.ndarray:
        """x + MoE(rms_norm(x)) on the device (the reference ``_moe_mlp_block``)."""
        if device_weights.backend != "rocm":
            raise RuntimeError("the MoE step needs the MI355X backend; got "
                               f"{device_weights.backend!r} device buffers")
        if device_weights.nbytes < layer.nbytes:
            raise RuntimeError(f"Layer {layer.layer_id}: device buffer size "
                               f"{device_weights.nbytes} < expected {layer.nbytes}")
        layout = self._layout(layer)
        cfg = self.moe_config(layout)
        desc = cfg.desc()
        if self._runner is None:
            self._runner = MoeRunner(backend)
        T = int(np.shape(x)[0])
        self._runner.reserve(desc, max(T, self.max_tokens, 1))
        weights = self._runner.bind(layout, int(device_weights.handle), stream)
        return self._runner.forward_numpy(desc, weights, x, stream)

    def moe_block_granular(self, layer: LayerSpec, x: np.ndarray, device_weights: DeviceBuffer,
                           backend: Any, stream: Any,
                           fetch: Callable[[list[int]], None]) -> np.ndarray:
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
        desc = self.moe_config(layout).desc()
        if self._runner is None:
            self._runner = MoeRunner(backend)
        T = int(np.shape(x)[0])
        self._runner.reserve(desc, max(T, self.max_tokens, 1))
        weights = self._runner.bind(layout, int(device_weights.handle), stream)
        active = self._runner.route_numpy(desc, weights, x, stream)
        fetch(active)
        return self._runner.finish_numpy(desc, weights, stream)

    def expert_ranges(self, layer: LayerSpec) -> tuple[list[tuple[int, int]], list[tuple[int, int]]]:
        """(core byte ranges, per-routed-expert byte ranges) of a packed MoE layer."""
        lay = self._layout(layer)
        return lay.core_ranges(layer.nbytes), lay.routed_expert_ranges()

    def run_layer_granular(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                           backend: Any, stream: Any, fetch: Callable[[list[int]], None]) -> Any:
        """``run_layer`` for a layer whose routed experts are copied on demand."""
        x = np.asarray(activations, dtype=np.float32)
        if self.attention is not None:
            x = self.attention(x, layer, device_weights, backend, stream)
        elif not self._moe_only(layer):
            raise NotImplementedError(
                "layer holds attention tensors; pass attention=... to run them")
        return self.moe_block_granular(layer, x, device_weights, backend, stream, fetch)

    def run_layer(self, layer: LayerSpec, activations: Any, device_weights: DeviceBuffer,
                  backend: Any, stream: Any) -> Any:
        x = np.asarray(activations, dtype=np.float32)
        if self.attention is not None:
            x = self.attention(x, layer, device_weights, backend, stream)
        elif not self._moe_only(layer):
            raise NotImplementedError(
                "layer holds attention tensors; pass attention=... to run them")
        if not layer.metadata.get("is_moe", True):
            raise NotImplementedError("dense MLP layers are not handled by this executor")
        return self.moe_block(layer, x, device_weights, backend, stream)

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


class Qwen3NextExecutor(_MoeExecutorBase):
    """Qwen3-Next (Qwen3NextForCausalLM): softmax router, renormalised top-k, no scaling,
    shared expert scaled by sigmoid(h . shared_expert_gate)."""

    _router_default = _lib.MX_ROUTER_SOFTMAX

    def __init__(self, config: dict[str, Any], **kw: Any) -> None:
        super().__init__(config, **kw)
        self.rms_norm_eps = float(config.get("rms_norm_eps", 1e-6))
        self.num_experts = int(config.get("num_experts", config.get("n_routed_experts", 512)))
        self.top_k = int(config.get("num_experts_per_tok", 10))
        self.norm_topk_prob = bool(config.get("norm_topk_prob", True))
        self.routed_scaling = 1.0
        self.num_experts_per_tok = self.top_k
