"""Pins of the linear-attention oracle (oracle/linear_attn_oracle.py) that need no GPU:
closed forms and library routines for each helper, and the reference's own outputs
(golden vectors) for the composed block."""
from __future__ import annotations

import json

import numpy as np
import pytest

from _cases import GOLDEN, digest
from moe_mi355x import synthetic as syn
from oracle import linear_attn_oracle as la


def test_softplus_known_values():
    x = np.array([-30.0, -1.0, 0.0, 1.0, 19.5, 20.0, 20.5, 80.0], np.float32)
    got = la.softplus(x)
    assert got[2] == np.float32(np.log(2.0))
    assert got[-1] == 80.0 and got[6] == np.float32(20.5)  # x > 20 passes through
    np.testing.assert_allclose(got[:6], np.logaddexp(0.0, x[:6].astype(np.float64)),
                               rtol=1e-6, atol=1e-12)


def test_causal_conv1d_matches_numpy_convolve():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((11, 5)).astype(np.float32)
    w = rng.standard_normal((5, 4)).astype(np.float32)
    got = la.causal_conv1d(x, w)
    for c in range(5):
        np.testing.assert_allclose(got[:, c], np.convolve(x[:, c], w[c])[:11], rtol=1e-5,
                                   atol=1e-6)
    # first tap weighs the current token: a unit impulse at t=0 returns the taps in order
    imp = np.zeros((6, 1), np.float32)
    imp[0] = 1.0
    assert np.array_equal(la.causal_conv1d(imp, np.array([[1., 2., 3., 4.]], np.float32))[:, 0],
                          np.array([1, 2, 3, 4, 0, 0], np.float32))
    # kernel longer than the sequence
    assert la.causal_conv1d(x[:2], w).shape == (2, 5)


def _closed_form(q, kb, v, g, n, dk, dv):
    """o_t = sum_{s<=t} exp(G_t - G_s) (kb_s . q_t) v_s with G the inclusive cumsum of g."""
    T = q.shape[0]
    q3 = q.reshape(T, n, dk).astype(np.float64)
    k3 = kb.reshape(T, n, dk).astype(np.float64)
    v3 = v.reshape(T, n, dv).astype(np.float64)
    G = np.cumsum(g.astype(np.float64), axis=0)  # [T, n]
    out = np.zeros((T, n, dv))
    for t in range(T):
        for s in range(t + 1):
            w = np.exp(G[t] - G[s]) * np.einsum("hk,hk->h", k3[s], q3[t])
            out[t] += w[:, None] * v3[s]
    return out.reshape(T, n * dv)


@pytest.mark.parametrize("n,dk,dv,T", [(2, 4, 4, 9), (3, 8, 4, 17), (1, 16, 8, 33)])
def test_recurrence_matches_closed_form(n, dk, dv, T):
    rng = np.random.default_rng(n * 100 + T)
    q = rng.standard_normal((T, n * dk)).astype(np.float32)
    kb = rng.standard_normal((T, n * dk)).astype(np.float32)
    v = rng.standard_normal((T, n * dv)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((T, n))) * 0.3).astype(np.float32)
    got = la.gated_recurrence(q, kb, v, g, n, dk, dv)
    ref = _closed_form(q, kb, v, g, n, dk, dv)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def test_recurrence_special_cases():
    rng = np.random.default_rng(5)
    n, dk, dv, T = 2, 4, 3, 6
    q = rng.standard_normal((T, n * dk)).astype(np.float32)
    kb = rng.standard_normal((T, n * dk)).astype(np.float32)
    v = rng.standard_normal((T, n * dv)).astype(np.float32)
    # one token: o = v (kb . q) per head
    o1 = la.gated_recurrence(q[:1], kb[:1], v[:1], np.zeros((1, n), np.float32), n, dk, dv)
    dots = np.einsum("hk,hk->h", kb[0].reshape(n, dk), q[0].reshape(n, dk))
    np.testing.assert_allclose(o1.reshape(n, dv), v[0].reshape(n, dv) * dots[:, None], rtol=1e-6)
    # no decay: plain causal linear attention  o_t = sum_{s<=t} v_s (kb_s . q_t)
    o = la.gated_recurrence(q, kb, v, np.zeros((T, n), np.float32), n, dk, dv)
    A = np.einsum("thk,shk->hts", q.reshape(T, n, dk), kb.reshape(T, n, dk))
    A = A * np.tril(np.ones((T, T)))[None]
    ref = np.einsum("hts,shv->thv", A, v.reshape(T, n, dv)).reshape(T, n * dv)
    np.testing.assert_allclose(o, ref, rtol=1e-5, atol=1e-5)
    # total decay (g = -inf): only the current token survives
    o_inf = la.gated_recurrence(q, kb, v, np.full((T, n), -np.inf, np.float32), n, dk, dv)
    cur = np.einsum("thk,thk->th", kb.reshape(T, n, dk), q.reshape(T, n, dk))
    np.testing.assert_allclose(o_inf, (v.reshape(T, n, dv) * cur[..., None]).reshape(T, -1),
                               rtol=1e-6)


def _golden_linear():
    path = GOLDEN / "linear_attn_index.json"
    return json.loads(path.read_text()) if path.exists() else {}


@pytest.mark.parametrize("name", sorted(_golden_linear()))
def test_oracle_matches_reference_golden(name):
    case = _golden_linear()[name]
    shape = syn.LinearAttnShape(**case["shape"])
    dt = np.dtype(case["dtype"])
    t = syn.make_linear_attn_tensors(shape, case["seed"], weight_dtype=dt, param_dtype=dt,
                                     norm_noise=case["norm_noise"])
    x = syn.make_inputs(case["seed"], case["tokens"], shape.hidden)
    assert digest(t) == case["tensors_sha256"] and digest({"x": x}) == case["x_sha256"]
    want = np.load(GOLDEN / f"{name}.npz")["out"]
    spec = la.LinearAttnSpec(shape.n_heads, shape.head_dim_k, shape.head_dim_v, shape.eps)
    got = la.linear_attn_block(x, t, spec)["out"]
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
