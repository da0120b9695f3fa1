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


def zipf_targets(tokens: int, n_experts: int, top_k: int, alpha: float = 1.1) -> np.ndarray:
    """Per-rank expert loads of a Zipf(alpha) skew over ``tokens * top_k`` routed pairs.

    p_r ∝ r^-alpha over ranks 1..E.  A token picks an expert at most once, so no load can
    exceed ``tokens``: loads above it are capped and the excess is shared among the
    uncapped ranks in proportion to p (repeated until no rank exceeds the cap).  The loads
    are then rounded to integers summing to ``tokens * top_k`` (largest remainders first).
    """
    E, total = n_experts, tokens * top_k
    if top_k > E:
        raise ValueError("top_k exceeds the expert count")
    p = np.arange(1, E + 1, dtype=np.float64) ** -alpha
    p /= p.sum()
    capped = np.zeros(E, dtype=bool)
    t = p * total
    while True:
        over = (t > tokens) & ~capped
        if not over.any():
            break
        capped |= over
        rest = total - tokens * int(capped.sum())
        t = np.where(capped, float(tokens), p / p[~capped].sum() * rest)
    loads = np.floor(t).astype(np.int64)
    frac = np.where(loads < tokens, t - loads, -1.0)
    loads[np.argsort(-frac, kind="stable")[: total - int(loads.sum())]] += 1
    return loads


def zipf_bias(logits: np.ndarray, top_k: int, alpha: float = 1.1, seed: int = 0,
              base_bias: np.ndarray | None = None, max_iters: int = 400
              ) -> tuple[np.ndarray, np.ndarray, dict]:
    """Per-expert correction bias that makes sigmoid-select routing of these tokens give
    Zipf(alpha) expert loads (``zipf_targets``, capped and renormalised).

    Experts get Zipf ranks from a seeded permutation.  With s = sigmoid(logits), token t
    selects expert e iff s[t, e] + b[e] is among its ``top_k`` largest keys, i.e. iff
    b[e] > theta[t, e] = (the k-th largest key of t among the other experts) - s[t, e].
    Given the other biases, the b[e] that gives expert e exactly its target load n_e lies
    between the n_e-th and (n_e + 1)-th smallest theta[:, e]; each sweep moves every b[e]
    halfway to the midpoint of that interval (all experts at once) and keeps the bias
    with the smallest L1 distance between realised and target loads.  Midpoints keep the
    selection away from the tie boundaries, so device logits (fp32 sums in another order)
    route the same way.  Returns (bias fp32, realised loads by expert id, info) with
    ``info`` = {"target": loads by expert id, "l1": L1 distance, "iters": sweeps run}.
    """
    T, E = logits.shape
    k = top_k
    rng = np.random.default_rng(seed)
    rank_of = np.empty(E, dtype=np.int64)
    rank_of[rng.permutation(E)] = np.arange(E)
    target = zipf_targets(T, E, k, alpha)[rank_of]
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    b = np.zeros(E) if base_bias is None else base_bias.astype(np.float64).copy()
    cols = np.arange(E)
    best = None
    it = 0
    for it in range(max_iters):
        bias32 = b.astype(np.float32)
        key = s + bias32.astype(np.float64)
        part = np.partition(-key, (k - 1, k), axis=1)
        kth, k1th = -part[:, k - 1], -part[:, k]
        chosen = key >= kth[:, None]
        loads = chosen.sum(axis=0)
        l1 = int(np.abs(loads - target).sum())
        if best is None or l1 < best[0]:
            best = (l1, bias32, loads)
        if l1 == 0:
            break
        theta = np.sort(np.where(chosen, k1th[:, None], kth[:, None]) - s, axis=0)
        lo = np.where(target > 0, theta[np.clip(target - 1, 0, T - 1), cols], theta[0] - 1e-3)
        hi = np.where(target < T, theta[np.clip(target, 0, T - 1), cols], theta[-1] + 1e-3)
        b += 0.5 * (0.5 * (lo + hi) - b)
    l1, bias32, loads = best
    return bias32, loads, {"target": target, "l1": l1, "iters": it + 1}


def zipf_summary(loads: np.ndarray, target: np.ndarray, tokens: int, top_k: int) -> dict:
    """Realised loads against the Zipf targets, with the workload's acceptance checks:
    every expert active, the hottest at >= 95 % of the token count, L1 distance <= 10 %
    of the routed pairs."""
    loads = np.asarray(loads, dtype=np.int64)
    srt = np.sort(loads)[::-1]
    l1 = int(np.abs(loads - np.asarray(target)).sum())
    out = {"n_active": int((loads > 0).sum()), "max_load": int(srt[0]),
           "min_load": int(srt[-1]), "median_load": float(np.median(srt)),
           "top5": srt[:5].tolist(), "target_top5": np.sort(target)[::-1][:5].tolist(),
           "l1": l1, "l1_frac": l1 / float(tokens * top_k)}
    out["ok"] = bool(out["n_active"] == loads.size and srt[0] >= 0.95 * tokens
                     and out["l1_frac"] <= 0.10)
    return out


def synthetic_host_params(shape: MoeShape, seed: int) -> dict[str, np.ndarray]:
    """Router weight and bias exactly as ``synthetic.make_tensors`` draws them (fp32)."""
    out = {"mlp.gate.weight": gen.normal(seed, stream_of("mlp.gate.weight"),
                                         (shape.n_experts, shape.hidden), std=0.02)}
    if shape.has_bias:
        out["mlp.gate.e_score_correction_bias"] = gen.normal(
            seed, stream_of("mlp.gate.e_score_correction_bias"), (shape.n_experts,), std=0.01)
    return out
