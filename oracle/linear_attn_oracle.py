"""CPU oracle of the Qwen3-Next linear-attention (Gated DeltaNet) block — TEST
INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker / the timed CPU baseline.  The product
(``moe_mi355x``, ``libmoe_mi355x.so``) never calls it; there is no CPU fallback.

A NumPy restatement of ``Qwen3NextExecutor._linear_attn_block``
(offload_runtime/executors/qwen3_next.py:207-269) and its helpers ``_softplus`` (:27-28),
``_sigmoid`` (:31-32), ``_causal_conv1d`` (:35-53) and ``_gated_delta_rule_recurrence``
(:56-95), with the primitives ``rms_norm`` / ``silu`` / ``linear_t`` of
offload_runtime/executors/_common.py:73-75, :83-84, :101-103.  Arithmetic is float32 with
fp16 tensors widened by NumPy promotion, as the reference does (``np.exp`` of an fp16
``A_log`` stays fp16, as there).

What the block computes, for T tokens, n heads (the reference reshapes q and k with the
value-head count, so it runs only when ``linear_num_key_heads == linear_num_value_heads``):
  h = rms_norm(x);  [q|k|v|z] = h W_qkvz^T;  [q|k|v] = silu(causal_conv1d([q|k|v]))
  [b|a] = h W_ba^T;  beta = sigmoid(b) (one per key channel);  g = -exp(A_log) softplus(a + dt_bias)
  per head: S_t = exp(g_t) S_{t-1} + v_t (beta_t k_t)^T,  o_t = S_t q_t   (S_0 = 0)
  out = x + (rms_norm(o) * silu(z)) W_out^T
The recurrence has no delta-rule correction term: this is what the reference executes.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np

from .moe_oracle import linear_t, rms_norm, sigmoid, silu

QKVZ = "linear_attn.in_proj_qkvz.weight"
BA = "linear_attn.in_proj_ba.weight"
CONV = "linear_attn.conv1d.weight"
A_LOG = "linear_attn.A_log"
DT_BIAS = "linear_attn.dt_bias"
OUT_NORM = "linear_attn.norm.weight"
OUT = "linear_attn.out_proj.weight"
IN_NORM = "input_layernorm.weight"


@dataclass(frozen=True)
class LinearAttnSpec:
    n_heads: int
    head_dim_k: int
    head_dim_v: int
    eps: float = 1e-6


def softplus(x: np.ndarray) -> np.ndarray:
    """qwen3_next.py:27-28: x where x > 20, else log1p(exp(x))."""
    return np.where(x > 20, x, np.log1p(np.exp(x)))


def causal_conv1d(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """qwen3_next.py:35-53: out[t, c] = sum_j x[t - j, c] w[c, j] (x[<0] = 0), summed
    j = 0, 1, ... in that order; w[:, 0] weighs the current token."""
    T, C = x.shape
    K = w.shape[-1]
    out = np.zeros_like(x)
    for j in range(K):
        if j < T:
            out[j:] += x[: T - j] * w[:, j]
    return out


def gated_recurrence(q: np.ndarray, kb: np.ndarray, v: np.ndarray, g: np.ndarray,
                     n: int, dk: int, dv: int) -> np.ndarray:
    """qwen3_next.py:56-95 with ``beta * k`` already formed (``kb``): per token
    S = S * exp(g_t)[h]; S += v_t[h, :, None] * kb_t[h, None, :]; o_t = S q_t."""
    T = q.shape[0]
    q3 = q.reshape(T, n, dk)
    k3 = kb.reshape(T, n, dk)
    v3 = v.reshape(T, n, dv)
    S = np.zeros((n, dv, dk), dtype=np.float32)
    out = np.zeros((T, n, dv), dtype=np.float32)
    for t in range(T):
        S = S * np.exp(g[t])[:, None, None]
        S = S + v3[t, :, :, None] * k3[t, :, None, :]
        out[t] = np.einsum("hvk,hk->hv", S, q3[t])
    return out.reshape(T, n * dv)


def linear_attn_block(x: np.ndarray, t: dict[str, np.ndarray], spec: LinearAttnSpec
                      ) -> dict[str, Any]:
    """qwen3_next.py:207-269; returns ``out`` and the intermediates the tests compare."""
    n, dk, dv = spec.n_heads, spec.head_dim_k, spec.head_dim_v
    qd, vd = n * dk, n * dv
    h = rms_norm(x, t[IN_NORM], spec.eps)
    qkvz = linear_t(h, t[QKVZ])
    q_raw, k_raw, v_raw, z = np.split(qkvz, [qd, 2 * qd, 2 * qd + vd], axis=-1)
    conv_w = t[CONV]
    if conv_w.ndim == 3:
        conv_w = conv_w.squeeze(1)
    conv = silu(causal_conv1d(np.concatenate([q_raw, k_raw, v_raw], axis=-1), conv_w))
    q, k, v = np.split(conv, [qd, 2 * qd], axis=-1)
    ba = linear_t(h, t[BA])
    beta_raw, a_raw = np.split(ba, [qd], axis=-1)
    beta = sigmoid(beta_raw)
    g = -np.exp(t[A_LOG]) * softplus(a_raw + t[DT_BIAS])
    kb = beta * k
    o = gated_recurrence(q, kb, v, g, n, dk, dv)
    gated = rms_norm(o, t[OUT_NORM], spec.eps) * silu(z)
    out = x + linear_t(gated, t[OUT])
    return {"h": h, "qkvz": qkvz, "ba": ba, "q": q, "kb": kb, "v": v, "g": g, "o": o,
            "gated": gated, "out": out.astype(np.float32)}
