"""Pins of the gated full-attention oracle (oracle/full_attn_oracle.py) that need no GPU:
closed forms for RoPE and the attention, causality, and the reference's own outputs
(golden vectors) for the composed block."""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

from _cases import GOLDEN, digest
from moe_mi355x import synthetic as syn
from oracle import full_attn_oracle as fa


def test_rope_is_a_complex_rotation():
    rng = np.random.default_rng(3)
    hd, T, base = 8, 5, 10000.0
    q = rng.standard_normal((2, T, hd)).astype(np.float32)
    k = rng.standard_normal((1, T, hd)).astype(np.float32)
    pos = np.arange(T, dtype=np.float32)
    rq, rk = fa.rope(q, k, pos, hd, base)
    half = hd // 2
    for x, r in ((q, rq), (k, rk)):
        z = x[..., :half].astype(np.complex128) + 1j * x[..., half:]
        th = np.outer(pos, base ** (-np.arange(half) / half))
        w = z * np.exp(1j * th)
        np.testing.assert_allclose(r[..., :half], w.real, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(r[..., half:], w.imag, rtol=1e-5, atol=1e-5)
        # position 0 is the identity; pair norms are preserved
        np.testing.assert_array_equal(r[:, 0], x[:, 0])
        np.testing.assert_allclose(np.abs(w), np.abs(z), rtol=1e-6)


def test_partial_rope_passes_the_tail_through():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 6, 16)).astype(np.float32)
    k = rng.standard_normal((2, 6, 16)).astype(np.float32)
    pos = np.arange(6, dtype=np.float32)
    pq, pk = fa.partial_rope(q, k, pos, 16, 4, 10000.0)
    np.testing.assert_array_equal(pq[..., 4:], q[..., 4:])
    np.testing.assert_array_equal(pk[..., 4:], k[..., 4:])
    rq, rk = fa.rope(q[..., :4], k[..., :4], pos, 4, 10000.0)
    np.testing.assert_array_equal(pq[..., :4], rq)


def test_attention_matches_brute_force():
    rng = np.random.default_rng(5)
    nh, T, hd = 3, 9, 8
    q = rng.standard_normal((nh, T, hd)).astype(np.float32)
    k = rng.standard_normal((nh, T, hd)).astype(np.float32)
    v = rng.standard_normal((nh, T, hd)).astype(np.float32)
    got = fa.attention(q, k, v, hd)
    ref = np.zeros((nh, T, hd))
    for h in range(nh):
        for t in range(T):
            s = np.array([q[h, t].astype(np.float64) @ k[h, j] for j in range(t + 1)]) / math.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref[h, t] = p @ v[h, : t + 1].astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_block_is_causal():
    shape = syn.FullAttnShape(64, 4, 2, 16, 0.25, 10000.0, 1e-6)
    t = syn.make_full_attn_tensors(shape, 9)
    spec = fa.FullAttnSpec(4, 2, 16, shape.rotary_dim, 10000.0, 1e-6)
    x = syn.make_inputs(9, 12, 64)
    a = fa.full_attn_block(x, t, spec)["out"]
    x2 = x.copy()
    x2[7:] += 1.0
    b = fa.full_attn_block(x2, t, spec)["out"]
    np.testing.assert_array_equal(a[:7], b[:7])
    assert not np.allclose(a[7:], b[7:])


def _golden():
    p = GOLDEN / "full_attn_index.json"
    return json.loads(p.read_text()) if p.exists() else {}


@pytest.mark.parametrize("name", sorted(_golden()))
def test_oracle_matches_reference_golden(name):
    case = _golden()[name]
    shape = syn.FullAttnShape(**case["shape"])
    dt = np.dtype(case["dtype"])
    t = syn.make_full_attn_tensors(shape, case["seed"], weight_dtype=dt, param_dtype=dt,
                                   norm_noise=case["norm_noise"])
    x = syn.make_inputs(case["seed"], case["tokens"], shape.hidden)
    assert digest(t) == case["tensors_sha256"] and digest({"x": x}) == case["x_sha256"]
    spec = fa.FullAttnSpec(shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.rotary_dim,
                           shape.rope_theta, shape.eps)
    got = fa.full_attn_block(x, t, spec)["out"]
    want = np.load(GOLDEN / f"{name}.npz")["out"]
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
