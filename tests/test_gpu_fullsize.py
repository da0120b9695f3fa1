"""Parity at the full benchmark shapes.

The whole batch runs on the GPU; the oracle then evaluates sampled tokens with only the
experts they route to (a token's MoE output depends on no other token), and the whole
batch is checked through properties that hold at any size: distinct expert ids per token,
per-expert counts equal to the histogram of the ids, routing weights summing to the routed
scaling, finite outputs, and the device's expert-sorted order being a stable permutation.
Bars as in test_gpu_parity: ids bit-exact on tokens whose selection margin clears fp32
noise, max abs error <= 2e-2 for fp16 / int8 weights against the fp32 evaluation.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.moe import read_device
from moe_mi355x.workloads import host_router_logits, synthetic_host_params, zipf_bias
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

SEED = 3131
LOWP_ABS = 2e-2
PROJ = ("gate_proj", "up_proj", "down_proj")


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def run_and_check(mi355x, stream, layer, shape, spec, mode_code, x, n_sample=4):
    T, k, E = x.shape[0], shape.top_k, shape.n_experts
    cfg = layer.config(top_k=k, router_mode=mode_code, routed_scaling=spec.routed_scaling,
                       eps=spec.eps, norm_topk_prob=spec.norm_topk_prob)
    out = layer.forward_numpy(cfg, x)
    v = layer.runner.views(cfg.desc(), T)
    ids = read_device(mi355x, v.topk_ids, np.int32, T * k, stream).reshape(T, k)
    w = read_device(mi355x, v.topk_w, np.float32, T * k, stream).reshape(T, k)
    counts = read_device(mi355x, v.counts, np.int32, E, stream)
    sorted_tok = read_device(mi355x, v.sorted_tok, np.int32, T * k, stream)
    offsets = read_device(mi355x, v.offsets, np.int32, E + 1, stream)
    # size-independent properties over the whole batch
    assert np.all(np.isfinite(out))
    assert all(len(set(r.tolist())) == k for r in ids), "repeated expert in a token"
    assert np.array_equal(counts, np.bincount(ids.ravel(), minlength=E))
    np.testing.assert_allclose(w.sum(axis=1), spec.routed_scaling, rtol=2e-5)
    for e in np.flatnonzero(counts)[:: max(1, E // 16)]:
        toks = sorted_tok[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(toks) > 0), f"expert {e}: rows not in ascending token order"
        assert np.all((ids[toks] == e).any(axis=1)), f"expert {e}: row of another expert"
    # sampled tokens against the oracle, with only their experts read back
    base = ["post_attention_layernorm.weight", "mlp.gate.weight"]
    base += [n for n in ("mlp.gate.e_score_correction_bias", "mlp.shared_expert_gate.weight")
             if n in layer.layout.entries]
    pre = layer.layout.shared_prefix
    base += [pre + p + ".weight" for p in PROJ] if pre else []
    t = layer.read_tensors(base)
    bias = t.get("mlp.gate.e_score_correction_bias")
    h = orc.rms_norm(x, t["post_attention_layernorm.weight"], spec.eps)
    margin = orc.topk_margin(orc.router_logits(h, t), bias, spec)
    ok = np.flatnonzero(margin > 1e-5)
    assert ok.size > 0.9 * T
    rng = np.random.default_rng(T)
    sample = np.sort(rng.choice(ok, size=min(n_sample, ok.size), replace=False))
    xs = x[sample]
    hs = orc.rms_norm(xs, t["post_attention_layernorm.weight"], spec.eps)
    ids_ref, _ = orc.route(orc.router_logits(hs, t), bias, spec)
    assert np.array_equal(ids[sample], ids_ref), "expert ids differ from the oracle"
    experts = sorted(set(ids_ref.ravel().tolist()))
    t.update(layer.read_tensors([f"mlp.experts.{e}.{p}.weight" for e in experts for p in PROJ]))
    ref = orc.moe_block(xs, t, spec)["out"]
    err = float(np.max(np.abs(out[sample] - ref)))
    say(f"    sampled tokens {sample.tolist()}: max abs err {err:.3e}")
    assert err <= LOWP_ABS


def test_glm47_prefill_2048_zipf_fp16_fragment_layout(mi355x, stream):
    say("[gpu] full size: GLM-4.7 fp16, 2048 tokens, Zipf routing, fragment layout")
    G = syn.GLM47
    x = syn.make_inputs(SEED, 2048, G.hidden)
    hp = synthetic_host_params(G, SEED)
    logits = host_router_logits(x, np.ones(G.hidden, np.float32), hp["mlp.gate.weight"], G.eps)
    bias, _, _ = zipf_bias(logits, G.top_k, 1.1, seed=SEED,
                           base_bias=hp["mlp.gate.e_score_correction_bias"])
    layer = DeviceMoeLayer.synthetic(mi355x, G, SEED, stream, weight_dtype="float16",
                                     param_dtype="float32", bias=bias).tile()
    try:
        spec = orc.MoeSpec(top_k=G.top_k, router_mode=orc.SIGMOID_SELECT_BIAS,
                           norm_topk_prob=True, routed_scaling=G.routed_scaling, eps=G.eps)
        run_and_check(mi355x, stream, layer, G, spec, _lib.MX_ROUTER_SIGMOID_SELECT_BIAS, x)
    finally:
        layer.close()


def test_qwen3next_4096_fp16_fragment_layout(mi355x, stream):
    say("[gpu] full size: Qwen3-Next fp16, 4096 tokens, fragment layout")
    Q = syn.QWEN3_NEXT
    x = syn.make_inputs(SEED + 1, 4096, Q.hidden)
    layer = DeviceMoeLayer.synthetic(mi355x, Q, SEED + 1, stream, weight_dtype="float16",
                                     param_dtype="float32").tile()
    try:
        spec = orc.MoeSpec(top_k=Q.top_k, router_mode=orc.SOFTMAX, norm_topk_prob=True,
                           routed_scaling=1.0, eps=Q.eps)
        run_and_check(mi355x, stream, layer, Q, spec, _lib.MX_ROUTER_SOFTMAX, x)
    finally:
        layer.close()


@pytest.mark.parametrize("T", [1, 16])
def test_glm47_decode_int8_loader_layout(mi355x, stream, T):
    say(f"[gpu] full size: GLM-4.7 per-row int8, {T} tokens, loader layout")
    G = syn.GLM47
    x = syn.make_inputs(SEED + 2 + T, T, G.hidden)
    layer = DeviceMoeLayer.synthetic(mi355x, G, SEED + 2, stream, weight_dtype="int8",
                                     param_dtype="float32")
    try:
        spec = orc.MoeSpec(top_k=G.top_k, router_mode=orc.SIGMOID_SELECT_BIAS,
                           norm_topk_prob=True, routed_scaling=G.routed_scaling, eps=G.eps)
        run_and_check(mi355x, stream, layer, G, spec, _lib.MX_ROUTER_SIGMOID_SELECT_BIAS, x,
                      n_sample=min(T, 6))
    finally:
        layer.close()
