"""Helpers shared by the test modules: golden cases and oracle specs."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from moe_mi355x import synthetic as syn
from oracle import moe_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def spec_for(shape: syn.MoeShape, router_mode: str | None = None) -> orc.MoeSpec:
    if shape.arch == syn.GLM:
        mode = router_mode or orc.REF_SOFTMAX_BIAS
        return orc.MoeSpec(top_k=shape.top_k, router_mode=mode, norm_topk_prob=True,
                           routed_scaling=shape.routed_scaling, eps=shape.eps)
    return orc.MoeSpec(top_k=shape.top_k, router_mode=router_mode or orc.SOFTMAX,
                       norm_topk_prob=True, routed_scaling=1.0, eps=shape.eps)


def digest(arrays: dict[str, np.ndarray]) -> str:
    h = hashlib.sha256()
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        h.update(name.encode())
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def golden_cases() -> dict[str, dict]:
    return json.loads((GOLDEN / "index.json").read_text())


def golden_case(name: str):
    """(shape, x, tensors, reference output) of a stored golden case."""
    c = golden_cases()[name]
    shape = syn.MoeShape(c["arch"], c["hidden"], c["n_experts"], c["top_k"], c["inter"],
                         c["shared_inter"], c["routed_scaling"], c["eps"], c["has_bias"],
                         c["has_shared_gate"])
    dt = np.dtype(c["dtype"])
    t = syn.make_tensors(shape, c["seed"], weight_dtype=dt, param_dtype=dt,
                         norm_noise=c["norm_noise"])
    x = syn.make_inputs(c["seed"], c["tokens"], shape.hidden)
    assert digest({"x": x}) == c["x_sha256"], f"{name}: regenerated x differs from the fixture"
    assert digest(t) == c["tensors_sha256"], f"{name}: regenerated tensors differ"
    ref = np.load(GOLDEN / f"{name}.npz")["out"]
    return shape, x, t, ref


def normwise_err(a: np.ndarray, ref: np.ndarray) -> float:
    """max |a - ref| / max |ref|."""
    den = float(np.max(np.abs(ref))) if ref.size else 1.0
    return float(np.max(np.abs(a.astype(np.float64) - ref.astype(np.float64)))) / max(den, 1e-30)
