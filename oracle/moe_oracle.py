"""CPU oracle of the MoE block — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker / the timed CPU baseline.  The product
(``moe_mi355x``, ``libmoe_mi355x.so``) never calls it; there is no CPU fallback.

A NumPy restatement of the reference hot path (haesookimDev/disk-mem-off):
  * ``GLM4MoeExecutor._moe_mlp_block``  offload_runtime/executors/glm4_moe.py:176-240
  * ``Qwen3NextExecutor._moe_mlp_block`` offload_runtime/executors/qwen3_next.py:273-333
  * primitives rms_norm / silu / softmax / linear_t  offload_runtime/executors/_common.py:73-75,
    :83-84, :87-90, :101-103; _sigmoid qwen3_next.py:31-32
  * host int8 dequantisation  offload_runtime/quantize.py:39-45
All arithmetic is float32 with fp16 weights widened by NumPy promotion, as the reference
does.  Int8 per-row experts are evaluated with their dequantised fp32 weights.

Two evaluation orders of the same mathematics:
  * ``moe_block_faithful`` keeps the reference's loop structure (one BLAS product per
    active expert in ``set`` order, per-token Python scatter).  It is the timed CPU
    baseline.
  * ``moe_block`` groups by expert with a stable dispatch and returns every intermediate
    (logits, ids, weights, counts, sorted order, per-row outputs) for the parity tests.

Router modes: ``ref_softmax_bias`` is what the reference executes (softmax over
logits + correction bias, glm4_moe.py:181-200); ``softmax`` is Qwen3-Next
(qwen3_next.py:278-293); ``sigmoid_select_bias`` is the GLM-4.5/4.7 checkpoint rule
(sigmoid scores, bias used only to select, weights from the unbiased scores), which the
reference does not implement — that mode differs from ``ref_softmax_bias`` only in the
router lines and is pinned by its own tests (see tests/test_oracle.py).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np

REF_SOFTMAX_BIAS = "ref_softmax_bias"
SIGMOID_SELECT_BIAS = "sigmoid_select_bias"
SOFTMAX = "softmax"

GLM_SHARED = "mlp.shared_experts."
QWEN_SHARED = "mlp.shared_expert."
SHARED_GATE = "mlp.shared_expert_gate.weight"


# ---- primitives ------------------------------------------------------------------------

def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """_common.py:73-75."""
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    return w * (x / rms)


def silu(x: np.ndarray) -> np.ndarray:
    """_common.py:83-84."""
    return x / (1.0 + np.exp(-x))


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """_common.py:87-90."""
    x_max = x.max(axis=axis, keepdims=True)
    e = np.exp(x - x_max)
    return e / e.sum(axis=axis, keepdims=True)


def sigmoid(x: np.ndarray) -> np.ndarray:
    """qwen3_next.py:31-32."""
    return 1.0 / (1.0 + np.exp(-x))


def linear_t(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """_common.py:101-103 (nn.Linear: x @ W.T)."""
    return x @ w.T


def dequant_int8_layer(raw: bytes, scale: float = 1.0, zero_point: int = 0) -> np.ndarray:
    """quantize.py:39-45: (int8 - zero_point) * scale -> float32."""
    q = np.frombuffer(raw, dtype=np.int8)
    return ((q.astype(np.float32) - zero_point) * scale).astype(np.float32)


def quantize_rows_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8: scale = fp16(max|W_row| / 127) (1 for a zero row),
    q = clip(rint(W / fp32(scale)), -127, 127).  The zero-point-0 per-row case of
    quantize.py:44."""
    w32 = np.asarray(w, dtype=np.float32)
    amax = np.abs(w32).max(axis=1)
    s = (amax / np.float32(127.0)).astype(np.float16)
    s[(amax == 0) | (s == 0)] = np.float16(1.0)
    q = np.clip(np.rint(w32 / s.astype(np.float32)[:, None]), -127, 127).astype(np.int8)
    return q, s


# ---- configuration ------------------------------------------------------------------------

@dataclass
class MoeSpec:
    """Executor config values used by the MoE block."""

    top_k: int
    router_mode: str = REF_SOFTMAX_BIAS
    norm_topk_prob: bool = True
    routed_scaling: float = 1.0
    eps: float = 1e-5


def weight(t: dict[str, np.ndarray], name: str) -> np.ndarray:
    """Tensor as the reference would consume it; per-row int8 is dequantised to fp32."""
    w = t[name]
    if w.dtype == np.int8:
        s = t[name + "_scale"].astype(np.float32)
        return w.astype(np.float32) * s[:, None]
    return w


def n_experts(t: dict[str, np.ndarray]) -> int:
    return int(t["mlp.gate.weight"].shape[0])


def shared_prefix(t: dict[str, np.ndarray]) -> str | None:
    for pre in (GLM_SHARED, QWEN_SHARED):
        if pre + "gate_proj.weight" in t:
            return pre
    return None


# ---- router ------------------------------------------------------------------------------

def router_logits(h: np.ndarray, t: dict[str, np.ndarray]) -> np.ndarray:
    """glm4_moe.py:181 / qwen3_next.py:278."""
    return h @ t["mlp.gate.weight"].T


def route(logits: np.ndarray, bias: np.ndarray | None, spec: MoeSpec
          ) -> tuple[np.ndarray, np.ndarray]:
    """Top-k ids (descending selection key) and routing weights.

    ref_softmax_bias: glm4_moe.py:182-200; softmax: qwen3_next.py:279-293 (pass
    routed_scaling=1); sigmoid_select_bias: sigmoid scores, top-k on score + bias,
    weights = unbiased scores, same renorm and scaling."""
    k = spec.top_k
    if spec.router_mode == SIGMOID_SELECT_BIAS:
        scores = sigmoid(logits)
        key = scores + bias if bias is not None else scores
        idx = np.argpartition(-key, k, axis=-1)[:, :k] if key.shape[-1] > k else \
            np.tile(np.arange(key.shape[-1]), (key.shape[0], 1))
        sel_key = np.take_along_axis(key, idx, axis=-1)
        order = np.argsort(-sel_key, axis=-1, kind="stable")
        idx = np.take_along_axis(idx, order, axis=-1)
    else:
        probs = _probs(logits, bias, spec)
        idx = np.argpartition(-probs, k, axis=-1)[:, :k] if probs.shape[-1] > k else \
            np.tile(np.arange(probs.shape[-1]), (probs.shape[0], 1))
        w = np.take_along_axis(probs, idx, axis=-1)
        order = np.argsort(-w, axis=-1)
        idx = np.take_along_axis(idx, order, axis=-1)
    return idx, route_weights(logits, bias, idx, spec)


def _probs(logits: np.ndarray, bias: np.ndarray | None, spec: MoeSpec) -> np.ndarray:
    """softmax(logits + bias) (glm4_moe.py:182-185) or softmax(logits) (qwen3_next.py:279)."""
    z = logits + bias if (spec.router_mode == REF_SOFTMAX_BIAS and bias is not None) \
        else logits
    return softmax(z, axis=-1)


def route_weights(logits: np.ndarray, bias: np.ndarray | None, ids: np.ndarray,
                  spec: MoeSpec) -> np.ndarray:
    """Routing weights of the experts ``ids`` [T, k] (in that slot order): the scores at
    those ids (softmax probabilities, or the unbiased sigmoid scores), renormalised over
    the k slots when norm_topk_prob (glm4_moe.py:198-199, + 1e-20) and times the routed
    scaling (glm4_moe.py:200).  ``route`` uses it on its own selection; the parity tests
    use it on a device selection that differs from ``route`` only between near-tied
    candidates."""
    if spec.router_mode == SIGMOID_SELECT_BIAS:
        w = np.take_along_axis(sigmoid(logits), ids, axis=-1)
    else:
        w = np.take_along_axis(_probs(logits, bias, spec), ids, axis=-1)
    if spec.norm_topk_prob:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return w * spec.routed_scaling


def selection_keys(logits: np.ndarray, bias: np.ndarray | None, spec: MoeSpec) -> np.ndarray:
    """The fp64 keys top-k ranks (an order-preserving image of each mode's key): sigmoid
    score + bias, logit + bias (softmax is monotonic), or the logit."""
    l64 = logits.astype(np.float64)
    b64 = None if bias is None else bias.astype(np.float64)
    if spec.router_mode == SIGMOID_SELECT_BIAS:
        return 1.0 / (1.0 + np.exp(-l64)) + (b64 if b64 is not None else 0.0)
    if spec.router_mode == REF_SOFTMAX_BIAS and b64 is not None:
        return l64 + b64
    return l64


def topk_margin(logits: np.ndarray, bias: np.ndarray | None, spec: MoeSpec) -> np.ndarray:
    """Per token, the fp64 gap between the k-th and (k+1)-th selection keys.  A token whose
    gap is below fp32 noise may legitimately select differently under another summation
    order of the router product."""
    s = -np.sort(-selection_keys(logits, bias, spec), axis=-1)
    k = spec.top_k
    if s.shape[-1] <= k:
        return np.full(s.shape[0], np.inf)
    return s[:, k - 1] - s[:, k]


def order_margin(logits: np.ndarray, bias: np.ndarray | None, spec: MoeSpec) -> np.ndarray:
    """Per token, the smallest fp64 gap between consecutive keys among the k + 1 largest:
    below fp32 noise, the selected set or the slot order of the ids may differ under
    another summation order of the router product."""
    s = -np.sort(-selection_keys(logits, bias, spec), axis=-1)
    n = min(spec.top_k + 1, s.shape[-1])
    if n < 2:
        return np.full(s.shape[0], np.inf)
    return np.min(s[:, : n - 1] - s[:, 1:n], axis=-1)


# ---- expert products ------------------------------------------------------------------------

def swiglu(x: np.ndarray, gate_w: np.ndarray, up_w: np.ndarray, down_w: np.ndarray) -> np.ndarray:
    """glm4_moe.py:222-224."""
    return linear_t(silu(linear_t(x, gate_w)) * linear_t(x, up_w), down_w)


def expert_act(x: np.ndarray, gate_w: np.ndarray, up_w: np.ndarray) -> np.ndarray:
    return silu(linear_t(x, gate_w)) * linear_t(x, up_w)


def shared_out(h: np.ndarray, t: dict[str, np.ndarray]) -> np.ndarray | None:
    """glm4_moe.py:234-238 / qwen3_next.py:321-331 (sigmoid gate when present)."""
    pre = shared_prefix(t)
    if pre is None:
        return None
    out = swiglu(h, weight(t, pre + "gate_proj.weight"), weight(t, pre + "up_proj.weight"),
                 weight(t, pre + "down_proj.weight"))
    if pre == QWEN_SHARED and SHARED_GATE in t:
        out = out * sigmoid(h @ t[SHARED_GATE].T)
    return out


# ---- dispatch ----------------------------------------------------------------------------

def dispatch(ids: np.ndarray, n_exp: int) -> dict[str, np.ndarray]:
    """Stable grouping of (token, slot) pairs by expert: the rows each expert gathers with
    h[token_mask] (glm4_moe.py:210-215), in ascending token order."""
    T, k = ids.shape
    flat = ids.reshape(-1)
    counts = np.bincount(flat, minlength=n_exp).astype(np.int32)
    offsets = np.zeros(n_exp + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    order = np.argsort(flat, kind="stable")  # pair index p = t*k + j, ascending t per expert
    sorted_tok = (order // k).astype(np.int32)
    pair_pos = np.empty(T * k, dtype=np.int32)
    pair_pos[order] = np.arange(T * k, dtype=np.int32)
    return {"counts": counts, "offsets": offsets, "sorted_tok": sorted_tok,
            "pair_pos": pair_pos.reshape(T, k), "order": order.astype(np.int32)}


# ---- the block ----------------------------------------------------------------------------

def moe_block_faithful(x: np.ndarray, t: dict[str, np.ndarray], spec: MoeSpec) -> np.ndarray:
    """The reference loop structure (glm4_moe.py:176-240 / qwen3_next.py:273-333)."""
    h = rms_norm(x, t["post_attention_layernorm.weight"], spec.eps)
    logits = router_logits(h, t)
    bias = t.get("mlp.gate.e_score_correction_bias")
    topk_indices, topk_weights = route(logits, bias, spec)
    output = np.zeros_like(h)
    for e in set(topk_indices.ravel().tolist()):
        mask = topk_indices == e
        token_mask = mask.any(axis=-1)
        if not token_mask.any():
            continue
        expert_out = swiglu(h[token_mask], weight(t, f"mlp.experts.{e}.gate_proj.weight"),
                            weight(t, f"mlp.experts.{e}.up_proj.weight"),
                            weight(t, f"mlp.experts.{e}.down_proj.weight"))
        for local_i, tok_i in enumerate(np.where(token_mask)[0]):
            w = topk_weights[tok_i][mask[tok_i]].sum()
            output[tok_i] += w * expert_out[local_i]
    so = shared_out(h, t)
    if so is not None:
        output = output + so
    return x + output


def moe_block(x: np.ndarray, t: dict[str, np.ndarray], spec: MoeSpec,
              ids: np.ndarray | None = None) -> dict[str, Any]:
    """Same mathematics as ``moe_block_faithful``, grouped by expert, with intermediates.

    Returns h, logits, ids, w, shared_w (1 or the Qwen sigmoid gate), the dispatch
    tables, act (per sorted row, routed rows then shared rows), y (weighted per-row
    outputs) and out = x + sum of the k routed rows + shared row.  ``ids`` [T, k], when
    given, replaces the top-k selection (weights from ``route_weights`` at those ids): the
    block evaluated on a selection that differs only between near-tied experts."""
    E = n_experts(t)
    h = rms_norm(x, t["post_attention_layernorm.weight"], spec.eps)
    logits = router_logits(h, t)
    bias = t.get("mlp.gate.e_score_correction_bias")
    if ids is None:
        ids, w = route(logits, bias, spec)
    else:
        ids = np.asarray(ids, dtype=np.int64)
        w = route_weights(logits, bias, ids, spec)
    d = dispatch(ids, E)
    T, k = ids.shape
    H = x.shape[1]
    pairs_w = w.reshape(-1)[d["order"]]
    acts, ys = [], []
    for e in range(E):
        lo, hi = int(d["offsets"][e]), int(d["offsets"][e + 1])
        if hi == lo:
            continue
        xe = h[d["sorted_tok"][lo:hi]]
        a = expert_act(xe, weight(t, f"mlp.experts.{e}.gate_proj.weight"),
                       weight(t, f"mlp.experts.{e}.up_proj.weight"))
        acts.append(a)
        ys.append(pairs_w[lo:hi, None] * linear_t(a, weight(t, f"mlp.experts.{e}.down_proj.weight")))
    act = np.concatenate(acts, axis=0) if acts else np.zeros((0, 0), np.float32)
    y = np.concatenate(ys, axis=0) if ys else np.zeros((0, H), np.float32)
    output = np.zeros_like(h)
    for j in range(k):
        output += y[d["pair_pos"][:, j]]
    pre = shared_prefix(t)
    shared_w = np.ones(T, dtype=np.float32)
    shared_act = None
    if pre is not None:
        shared_act = expert_act(h, weight(t, pre + "gate_proj.weight"),
                                weight(t, pre + "up_proj.weight"))
        so = linear_t(shared_act, weight(t, pre + "down_proj.weight"))
        if pre == QWEN_SHARED and SHARED_GATE in t:
            g = sigmoid(h @ t[SHARED_GATE].T)
            shared_w = g[:, 0].astype(np.float32)
            so = so * g
        output = output + so
    return {"h": h, "logits": logits, "ids": ids.astype(np.int32), "w": w.astype(np.float32),
            "shared_w": shared_w, "act": act, "shared_act": shared_act, "y": y,
            "out": x + output, **d}
