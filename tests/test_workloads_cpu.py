"""Algorithmic byte / FLOP accounting used by the roofline entries, checked against the
closed forms of the GLM-4.7 decode and Qwen3-Next workloads."""
from __future__ import annotations

import numpy as np

from moe_mi355x import synthetic as syn
from moe_mi355x.workloads import call_traffic, expert_bytes, zipf_bias


def test_expert_bytes():
    gu, dn = expert_bytes(syn.GLM47, "float16", 1536)
    assert gu + dn == 3 * 1536 * 5120 * 2 == 47_185_920
    gu8, dn8 = expert_bytes(syn.GLM47, "int8", 1536)
    assert gu8 + dn8 == 23_592_960 + (2 * 1536 + 5120) * 2


def test_glm_decode_t1_layer_bytes():
    tr = call_traffic(syn.GLM47, "float16", 1, 8)
    # (8 routed + 1 shared) x 47.19 MB + fp32 router 160 x 5120 x 4 + x and out
    assert tr["layer_bytes"] == 9 * 47_185_920 + 160 * 5120 * 4 + 2 * 5120 * 4
    assert tr["layer_flops"] == 2 * 5120 * 160 + 2 * 3 * 5120 * 1536 * 9


def test_qwen_t1_layer_bytes():
    tr = call_traffic(syn.QWEN3_NEXT, "float16", 1, 10)
    assert tr["layer_bytes"] == 11 * 6_291_456 + 512 * 2048 * 4 + 2 * 2048 * 4


def test_zipf_targets_capped_and_renormalised():
    from moe_mi355x.workloads import zipf_targets

    T, E, k, a = 2048, 160, 8, 1.1
    t = zipf_targets(T, E, k, a)
    assert t.sum() == T * k and t.max() == T and np.all(np.diff(t) <= 0)
    # the GLM-4.7 prefill: one capped rank, the rest Zipf(1.1) over the remaining pairs
    assert t[:3].tolist() == [2048, 1875, 1200] and t[-1] == 15
    p = np.arange(1, E + 1, dtype=np.float64) ** -a
    want = p[1:] / p[1:].sum() * (T * k - T)
    assert np.all(np.abs(t[1:] - want) < 1.0)
    # no cap needed: plain rounding of T k p
    t2 = zipf_targets(10000, 16, 2, 1.1)
    p16 = np.arange(1, 17, dtype=np.float64) ** -1.1
    assert t2.sum() == 20000 and np.all(np.abs(t2 - 20000 * p16 / p16.sum()) < 1.0)


def test_zipf_bias_realises_targets():
    from moe_mi355x.workloads import zipf_summary

    rng = np.random.default_rng(0)
    T, E, k = 512, 40, 4
    logits = rng.standard_normal((T, E)).astype(np.float32) * 1.4
    bias, loads, info = zipf_bias(logits, k, 1.1, seed=1)
    assert bias.dtype == np.float32 and loads.sum() == T * k
    # brute force: the fp32 bias routes every token to the loads reported
    key = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias.astype(np.float64)
    ids = np.argsort(-key, axis=1, kind="stable")[:, :k]
    assert np.array_equal(np.bincount(ids.ravel(), minlength=E), loads)
    z = zipf_summary(loads, info["target"], T, k)
    assert z["ok"] and z["max_load"] == T and z["n_active"] == E
    assert info["l1"] == z["l1"] and z["l1_frac"] <= 0.02


def test_zipf_summary_flags_a_weak_skew():
    from moe_mi355x.workloads import zipf_summary, zipf_targets

    tgt = zipf_targets(2048, 160, 8)
    flat = np.full(160, 2048 * 8 // 160)
    z = zipf_summary(flat, tgt, 2048, 8)
    assert not z["ok"] and z["max_load"] < 0.95 * 2048
