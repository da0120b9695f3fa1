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


def test_zipf_bias_skews_loads():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((2048, 40)).astype(np.float32) * 0.3
    bias, loads, c = zipf_bias(logits, 4, 1.1, seed=1)
    assert loads.sum() == 2048 * 4 and c > 0
    srt = np.sort(loads)[::-1]
    assert srt[0] > 4 * np.median(srt)
