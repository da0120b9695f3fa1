"""CPU oracle of the Qwen3-Next gated full-attention block — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker / the timed CPU baseline.  The product
(``moe_mi355x``, ``libmoe_mi355x.so``) never calls it; there is no CPU fallback.

A NumPy restatement of ``Qwen3NextExecutor._full_attn_block``
(offload_runtime/executors/qwen3_next.py:161-205) with the helpers of
offload_runtime/executors/_common.py: ``rope`` (:105-127), ``repeat_kv`` (:130-134),
``rms_norm_no_weight`` (:137-140), ``partial_rope`` (:143-153), ``rms_norm`` (:73-75),
``softmax`` (:87-90) and ``linear_t`` (:101-103).  Arithmetic is float32 (RoPE frequencies
and angles in float64, rounded to float32 before cos / sin), as in the reference.

  h = rms_norm(x);  [q | gate] = h W_q^T (halves);  k = h W_k^T;  v = h W_v^T
  per head: q = rms_norm_no_weight(q) * q_norm;  k likewise;  RoPE on the first
  rotary_dim = int(head_dim * partial_rotary_factor) dims (rotate-half form)
  attention: softmax((q k^T) / sqrt(head_dim) + causal mask(-1e10)) v, key/value heads
  repeated n_heads / n_kv_heads times;  out = x + (attn * sigmoid(gate)) W_o^T
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import numpy as np

from .moe_oracle import linear_t, rms_norm, sigmoid, softmax

IN_NORM = "input_layernorm.weight"
Q = "self_attn.q_proj.weight"
K = "self_attn.k_proj.weight"
V = "self_attn.v_proj.weight"
O = "self_attn.o_proj.weight"
Q_NORM = "self_attn.q_norm.weight"
K_NORM = "self_attn.k_norm.weight"


@dataclass(frozen=True)
class FullAttnSpec:
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rotary_dim: int
    rope_theta: float = 5000000.0
    eps: float = 1e-6


def rms_norm_no_weight(x: np.ndarray, eps: float) -> np.ndarray:
    """_common.py:137-140."""
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    return x / rms


def rope(q: np.ndarray, k: np.ndarray, positions: np.ndarray, head_dim: int,
         base: float) -> tuple[np.ndarray, np.ndarray]:
    """_common.py:105-127: rotate-half RoPE over the last head_dim dims."""
    half = head_dim // 2
    freqs = 1.0 / (base ** (np.arange(0, half, dtype=np.float64) / half))
    ang = np.outer(positions.astype(np.float64), freqs).astype(np.float32)
    c, s = np.cos(ang), np.sin(ang)

    def rot(x):
        x1, x2 = x[..., :half], x[..., half:]
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)

    return rot(q), rot(k)


def partial_rope(q, k, positions, head_dim, rotary_dim, base):
    """_common.py:143-153: RoPE on the first rotary_dim dims, the rest passed through."""
    qr, qp = q[..., :rotary_dim], q[..., rotary_dim:]
    kr, kp = k[..., :rotary_dim], k[..., rotary_dim:]
    qr, kr = rope(qr, kr, positions, rotary_dim, base)
    return np.concatenate([qr, qp], axis=-1), np.concatenate([kr, kp], axis=-1)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, head_dim: int) -> np.ndarray:
    """qwen3_next.py:190-198 on [heads, T, hd] inputs (k, v already repeated)."""
    T = q.shape[1]
    scores = (q @ k.transpose(0, 2, 1)) / math.sqrt(head_dim)
    mask = np.triu(np.full((T, T), -1e10, dtype=np.float32), k=1)
    return softmax(scores + mask, axis=-1) @ v


def full_attn_block(x: np.ndarray, t: dict[str, np.ndarray], spec: FullAttnSpec
                    ) -> dict[str, Any]:
    """qwen3_next.py:161-205; returns ``out`` and intermediates."""
    T = x.shape[0]
    nh, nkv, hd = spec.n_heads, spec.n_kv_heads, spec.head_dim
    h = rms_norm(x, t[IN_NORM], spec.eps)
    qg = linear_t(h, t[Q])
    q, gate = np.split(qg, 2, axis=-1)
    k = linear_t(h, t[K])
    v = linear_t(h, t[V])
    q = q.reshape(T, nh, hd).transpose(1, 0, 2)
    k = k.reshape(T, nkv, hd).transpose(1, 0, 2)
    v = v.reshape(T, nkv, hd).transpose(1, 0, 2)
    if Q_NORM in t:
        q = rms_norm_no_weight(q, spec.eps) * t[Q_NORM]
    if K_NORM in t:
        k = rms_norm_no_weight(k, spec.eps) * t[K_NORM]
    pos = np.arange(T, dtype=np.float32)
    if spec.rotary_dim < hd:
        q, k = partial_rope(q, k, pos, hd, spec.rotary_dim, spec.rope_theta)
    else:
        q, k = rope(q, k, pos, hd, spec.rope_theta)
    rep = nh // nkv
    kr = np.repeat(k, rep, axis=0) if rep > 1 else k
    vr = np.repeat(v, rep, axis=0) if rep > 1 else v
    att = attention(q, kr, vr, hd)
    att = att.transpose(1, 0, 2).reshape(T, nh * hd)
    gated = att * sigmoid(gate)
    out = x + linear_t(gated, t[O])
    return {"h": h, "qg": qg, "q": q, "k": k, "v": v, "att": att, "gated": gated,
            "out": out.astype(np.float32)}
