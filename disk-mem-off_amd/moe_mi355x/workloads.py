"""Benchmark workload helpers: algorithmic bytes / FLOPs of one MoE-block call and the
Zipf-skewed router bias used for the prefill workload.

Algorithmic traffic of one call (what an ideal kernel must move through HBM):
  expert weights of every distinct expert the tokens route to, plus the shared expert,
  each read once (gate + up + down, plus the fp16 row scales for int8), the router
  weight, the fp32 input and output activations.
FLOPs: 2 T H E (router) + 2 * 3 * H * I per routed (token, slot) pair and per token for
the shared expert.
"""
from __future__ import annotations

import numpy as np

from . import gen
from .synthetic import MoeShape, stream_of

HBM_PEAK = 8.0e12         # MI355X HBM3E, bytes/s
MFMA_F16_PEAK = 2.5e15    # MI355X dense fp16 MFMA, FLOP/s
MFMA_F32_PEAK = 157.3e12  # MI355X fp32 matrix, FLOP/s

ESZ = {"float32": 4, "float16": 2, "int8": 1}


def expert_bytes(shape: MoeShape, wdt: str, inter: int) -> tuple[int, int]:
    """(gate + up bytes, down bytes) of one expert with intermediate size ``inter``."""
    e = ESZ[wdt]
    gu = 2 * inter * shape.hidden * e
    dn = shape.hidden * inter * e
    if wdt == "int8":
        gu += 2 * inter * 2
        dn += shape.hidden * 2
    return gu, dn


def call_traffic(shape: MoeShape, wdt: str, tokens: int, n_active: int,
                 param_bytes: int = 4) -> dict[str, float]:
    """Algorithmic bytes and FLOPs of one block call with ``n_active`` routed experts."""
    H, E, k = shape.hidden, shape.n_experts, shape.top_k
    gu, dn = expert_bytes(shape, wdt, shape.inter)
    sgu, sdn = expert_bytes(shape, wdt, shape.shared_inter) if shape.shared_inter else (0, 0)
    R = tokens * k + (tokens if shape.shared_inter else 0)
    imax = max(shape.inter, shape.shared_inter)
    aesz = 4 if wdt == "float32" else 2
    gate_up = n_active * gu + sgu + tokens * H * aesz + R * imax * aesz
    down = n_active * dn + sdn + R * imax * aesz + R * H * 4
    layer = n_active * (gu + dn) + sgu + sdn + E * H * param_bytes + 2 * tokens * H * 4
    flops_router = 2.0 * tokens * H * E
    flops_routed = 2.0 * 3 * H * shape.inter * tokens * k
    flops_shared = 2.0 * 3 * H * shape.shared_inter * tokens
    return {"gate_up_bytes": float(gate_up), "down_bytes": float(down),
            "layer_bytes": float(layer),
            "gate_up_flops": (flops_routed + flops_shared) * 2 / 3,
            "down_flops": (flops_routed + flops_shared) / 3,
            "layer_flops": flops_router + flops_routed + flops_shared}


def host_router_logits(x: np.ndarray, norm_w: np.ndarray, router_w: np.ndarray,
                       eps: float) -> np.ndarray:
    """Router logits on the host (only used to shape the synthetic prefill workload)."""
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    h = norm_w * (x / rms)
    return h @ router_w.T


def zipf_bias(logits: np.ndarray, top_k: int, alpha: float = 1.1, seed: int = 0,
              base_bias: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray, float]:
    """Correction bias that skews sigmoid-select routing towards Zipf(alpha) expert loads.

    Experts get ranks from a seeded permutation; bias_e = c * log(p_rank(e)) with
    p_r ∝ r^-alpha.  ``c`` is chosen on a grid to minimise the L1 distance between the
    realised per-rank loads and the Zipf targets capped at T (a token picks an expert at
    most once).  Returns (bias, realised loads by expert id, c)."""
    T, E = logits.shape
    rng = np.random.default_rng(seed)
    rank_of = np.empty(E, dtype=np.int64)
    rank_of[rng.permutation(E)] = np.arange(E)
    p = (np.arange(1, E + 1, dtype=np.float64)) ** -alpha
    p /= p.sum()
    target = np.minimum(p * T * top_k, T)
    scores = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    b0 = np.zeros(E) if base_bias is None else base_bias.astype(np.float64)
    best = None
    for c in np.linspace(0.0, 0.3, 61):
        bias = b0 + c * np.log(p[rank_of])
        key = scores + bias
        ids = np.argpartition(-key, top_k, axis=-1)[:, :top_k]
        loads = np.bincount(ids.ravel(), minlength=E)
        err = np.abs(loads[np.argsort(rank_of)] - target).sum()
        if best is None or err < best[0]:
            best = (err, bias, loads, c)
    _, bias, loads, c = best
    return bias.astype(np.float32), loads, float(c)


def synthetic_host_params(shape: MoeShape, seed: int) -> dict[str, np.ndarray]:
    """Router weight and bias exactly as ``synthetic.make_tensors`` draws them (fp32)."""
    out = {"mlp.gate.weight": gen.normal(seed, stream_of("mlp.gate.weight"),
                                         (shape.n_experts, shape.hidden), std=0.02)}
    if shape.has_bias:
        out["mlp.gate.e_score_correction_bias"] = gen.normal(
            seed, stream_of("mlp.gate.e_score_correction_bias"), (shape.n_experts,), std=0.01)
    return out
