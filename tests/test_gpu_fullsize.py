"""Parity at the full benchmark shapes, with the benchmark's own seeds and layouts.

Every test runs a whole batch on the GPU and then checks, over the whole batch, the
routing against the oracle evaluated on the host from the layer's own router tensors
(tests/_routing.py: ids of every clear token, weights at the device ids, and the integer
dispatch tables — counts, offsets, expert-sorted order, inverse permutation, shared rows —
bit for bit).  Outputs of every token are then checked against the oracle evaluated with
the experts the batch routes to, read back from the device, so every m-tile of the prefill
launches (each expert-sorted row) is compared, at 2048 and 4096 tokens too.

Bars as in test_gpu_parity: fp16 / int8 weights, max abs error <= 2e-2 against the fp32
evaluation with the same (dequantised) weights.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from _routing import check_routing_tables
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.moe import read_device
from moe_mi355x.workloads import (host_router_logits, synthetic_host_params, zipf_bias,
                                  zipf_summary)
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

LOWP_ABS = 2e-2
PROJ = ("gate_proj", "up_proj", "down_proj")
# Seeds of the benchmark workloads (bench.py): the layers and the decode inputs.
BENCH_SEED = 2026
HEADLINE_T = 32


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def glm_spec() -> orc.MoeSpec:
    G = syn.GLM47
    return orc.MoeSpec(top_k=G.top_k, router_mode=orc.SIGMOID_SELECT_BIAS, norm_topk_prob=True,
                       routed_scaling=G.routed_scaling, eps=G.eps)


def qwen_spec() -> orc.MoeSpec:
    Q = syn.QWEN3_NEXT
    return orc.MoeSpec(top_k=Q.top_k, router_mode=orc.SOFTMAX, norm_topk_prob=True,
                       routed_scaling=1.0, eps=Q.eps)


def bench_inputs(T: int, hidden: int) -> np.ndarray:
    """The benchmark's decode inputs: the headline batch uses the layer seed itself."""
    return syn.make_inputs(BENCH_SEED if T == HEADLINE_T else BENCH_SEED + T, T, hidden)


def run_and_check(mi355x, stream, layer, shape, spec, mode_code, x, sample=None):
    """Forward the whole batch, check its routing over every token and the outputs of
    ``sample`` (all tokens when None)."""
    T, k, E = x.shape[0], shape.top_k, shape.n_experts
    has_sh = shape.shared_inter > 0
    R = T * k + (T if has_sh else 0)
    cfg = layer.config(top_k=k, router_mode=mode_code, routed_scaling=spec.routed_scaling,
                       eps=spec.eps, norm_topk_prob=spec.norm_topk_prob)
    out = layer.forward_numpy(cfg, x)
    assert np.all(np.isfinite(out)), "non-finite output"
    v = layer.runner.views(cfg.desc(), T)
    dev = {
        "ids": read_device(mi355x, v.topk_ids, np.int32, T * k, stream).reshape(T, k),
        "w": read_device(mi355x, v.topk_w, np.float32, T * k, stream).reshape(T, k),
        "shared_w": read_device(mi355x, v.shared_w, np.float32, T, stream),
        "counts": read_device(mi355x, v.counts, np.int32, E, stream),
        "offsets": read_device(mi355x, v.offsets, np.int32, E + 1, stream),
        "sorted_tok": read_device(mi355x, v.sorted_tok, np.int32, R, stream),
        "pair_pos": read_device(mi355x, v.pair_pos, np.int32, T * k, stream).reshape(T, k),
        "n_groups": int(read_device(mi355x, v.n_groups, np.int32, 1, stream)[0]),
    }
    base = ["post_attention_layernorm.weight", "mlp.gate.weight"]
    base += [n for n in ("mlp.gate.e_score_correction_bias", "mlp.shared_expert_gate.weight")
             if n in layer.layout.entries]
    pre = layer.layout.shared_prefix
    base += [pre + p + ".weight" for p in PROJ] if pre else []
    t = layer.read_tensors(base)
    bias = t.get("mlp.gate.e_score_correction_bias")
    h = orc.rms_norm(x, t["post_attention_layernorm.weight"], spec.eps)
    logits = orc.router_logits(h, t)
    label = f"{shape.arch} T={T}"
    check_routing_tables(dev, logits, bias, spec, E, label, has_shared=has_sh)
    n_active = len(np.unique(dev["ids"]))
    assert dev["n_groups"] == n_active + (1 if has_sh else 0)
    if "mlp.shared_expert_gate.weight" in t:
        g = orc.sigmoid(h @ t["mlp.shared_expert_gate.weight"].T)[:, 0]
        np.testing.assert_allclose(dev["shared_w"], g, rtol=1e-5, atol=1e-7)
    rows = np.arange(T) if sample is None else np.asarray(sample)
    ids = dev["ids"][rows]
    experts = sorted(set(ids.ravel().tolist()))
    t.update(layer.read_tensors([f"mlp.experts.{e}.{p}.weight" for e in experts for p in PROJ]))
    ref = orc.moe_block(x[rows], Fp32Weights(t), spec, ids=ids)["out"]
    err = float(np.max(np.abs(out[rows] - ref)))
    say(f"    {label}: {n_active} routed experts, outputs of {rows.size} tokens: max abs err "
        f"{err:.3e}")
    assert err <= LOWP_ABS
    return dev["counts"]


class Fp32Weights(dict):
    """Tensors with fp16 entries widened to fp32 when the oracle reads them: the values
    NumPy's promotion gives, through BLAS (a whole 2048-token GLM-4.7 batch in seconds
    instead of the promotion loop's minutes)."""

    def __getitem__(self, name):
        v = dict.__getitem__(self, name)
        return v.astype(np.float32) if v.dtype == np.float16 else v


# ---- GLM-4.7 fp16, fragment layout: the benchmark layer -------------------------------------

@pytest.fixture(scope="module")
def glm47_fp16(mi355x, stream):
    say("[gpu] full size: building the GLM-4.7 fp16 layer (fragment layout)")
    layer = DeviceMoeLayer.synthetic(mi355x, syn.GLM47, BENCH_SEED, stream,
                                     weight_dtype="float16", param_dtype="float32").tile()
    yield layer
    layer.close()


@pytest.mark.parametrize("T", [1, 8, 32])
def test_glm47_decode_fp16_fragment_layout(mi355x, stream, glm47_fp16, T):
    """The decode benchmark batches: one token (experts selected inside the gate/up
    launch), 8 tokens (4-way K split of the single-m-frag gate/up), 32 (the headline)."""
    say(f"[gpu] full size: GLM-4.7 fp16 decode, {T} tokens, fragment layout")
    run_and_check(mi355x, stream, glm47_fp16, syn.GLM47, glm_spec(),
                  _lib.MX_ROUTER_SIGMOID_SELECT_BIAS, bench_inputs(T, syn.GLM47.hidden))


def test_glm47_prefill_2048_zipf_fp16_fragment_layout(mi355x, stream, glm47_fp16):
    """The prefill benchmark: the same layer with the correction bias replaced by the
    Zipf(1.1) skew (hot experts of several 128-row m-tiles), 2048 tokens."""
    say("[gpu] full size: GLM-4.7 fp16, 2048 tokens, Zipf routing, fragment layout")
    G = syn.GLM47
    layer = glm47_fp16
    x = syn.make_inputs(BENCH_SEED + 1, 2048, G.hidden)
    hp = synthetic_host_params(G, BENCH_SEED)
    logits = host_router_logits(x, np.ones(G.hidden, np.float32), hp["mlp.gate.weight"], G.eps)
    bias, loads, info = zipf_bias(logits, G.top_k, 1.1, seed=BENCH_SEED,
                                  base_bias=hp["mlp.gate.e_score_correction_bias"])
    z = zipf_summary(loads, info["target"], 2048, G.top_k)
    say(f"    Zipf(1.1) loads on the host: {z}")
    assert z["ok"], "the bias must realise the capped Zipf(1.1) loads"
    off = layer.layout.offset("mlp.gate.e_score_correction_bias")
    orig = layer.read("mlp.gate.e_score_correction_bias")
    try:
        layer.write(off, bias)
        dev_counts = run_and_check(mi355x, stream, layer, G, glm_spec(),
                                   _lib.MX_ROUTER_SIGMOID_SELECT_BIAS, x)
        zd = zipf_summary(dev_counts, info["target"], 2048, G.top_k)
        say(f"    Zipf(1.1) loads on the device: {zd}")
        assert zd["ok"]
    finally:
        layer.write(off, orig)


# ---- Qwen3-Next fp16, fragment layout ---------------------------------------------------------

@pytest.fixture(scope="module")
def qwen3next_fp16(mi355x, stream):
    say("[gpu] full size: building the Qwen3-Next fp16 layer (fragment layout)")
    layer = DeviceMoeLayer.synthetic(mi355x, syn.QWEN3_NEXT, BENCH_SEED, stream,
                                     weight_dtype="float16", param_dtype="float32").tile()
    yield layer
    layer.close()


def test_qwen3next_one_token_fp16_fragment_layout(mi355x, stream, qwen3next_fp16):
    """One token over 512 experts: the gate/up launch selects with 4 waves of 128 experts."""
    say("[gpu] full size: Qwen3-Next fp16, 1 token, fragment layout")
    Q = syn.QWEN3_NEXT
    run_and_check(mi355x, stream, qwen3next_fp16, Q, qwen_spec(), _lib.MX_ROUTER_SOFTMAX,
                  syn.make_inputs(BENCH_SEED + 1, 1, Q.hidden))


def test_qwen3next_4096_fp16_fragment_layout(mi355x, stream, qwen3next_fp16):
    say("[gpu] full size: Qwen3-Next fp16, 4096 tokens, fragment layout")
    Q = syn.QWEN3_NEXT
    run_and_check(mi355x, stream, qwen3next_fp16, Q, qwen_spec(), _lib.MX_ROUTER_SOFTMAX,
                  syn.make_inputs(BENCH_SEED + 4096, 4096, Q.hidden))


# ---- GLM-4.7 per-row int8, both layouts ---------------------------------------------------------

@pytest.mark.parametrize("layout", ["rows", "frag16"])
@pytest.mark.parametrize("T", [1, 16])
def test_glm47_decode_int8(mi355x, stream, T, layout):
    say(f"[gpu] full size: GLM-4.7 per-row int8, {T} tokens, {layout} layout")
    G = syn.GLM47
    layer = DeviceMoeLayer.synthetic(mi355x, G, BENCH_SEED, stream, weight_dtype="int8",
                                     param_dtype="float32")
    if layout == "frag16":
        layer.tile()
    try:
        run_and_check(mi355x, stream, layer, G, glm_spec(), _lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
                      syn.make_inputs(BENCH_SEED + T, T, G.hidden))
    finally:
        layer.close()
