"""GPU parity of the MoE hot path against the oracle and the reference golden vectors.

Bars: expert ids and per-expert token counts bit-exact (tokens whose k-th/(k+1)-th key gap
is below fp32 noise are reported, never silently excused); fp32 weights: normwise
relative error <= 1e-4; fp16 / int8 weights: max abs error <= 2e-2 against the fp32
evaluation with the same (dequantised) weights.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from _cases import golden_case, golden_cases, normwise_err, spec_for
from _routing import check_routing_tables
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.moe import read_device
from moe_mi355x.quantize import quantize_moe_tensors
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

FP32_REL = 1e-4
LOWP_ABS = 2e-2

MODE_CODE = {orc.REF_SOFTMAX_BIAS: _lib.MX_ROUTER_REF_SOFTMAX_BIAS,
             orc.SIGMOID_SELECT_BIAS: _lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
             orc.SOFTMAX: _lib.MX_ROUTER_SOFTMAX}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def run_device(mi355x, stream, tensors, shape, spec, x, frag=False):
    """Forward on the device (expert weights re-laid in MX_LAYOUT_FRAG16 when ``frag``);
    returns (out, views dict)."""
    dl = DeviceMoeLayer.from_host(mi355x, tensors, stream)
    try:
        if frag:
            dl.tile()
        cfg = dl.config(top_k=spec.top_k, router_mode=MODE_CODE[spec.router_mode],
                        routed_scaling=spec.routed_scaling, eps=spec.eps,
                        norm_topk_prob=spec.norm_topk_prob)
        out = dl.forward_numpy(cfg, x)
        T, k, E = x.shape[0], spec.top_k, shape.n_experts
        v = dl.runner.views(cfg.desc(), T)
        has_sh = cfg.shared_inter > 0
        R = T * k + (T if has_sh else 0)
        views = {
            "ids": read_device(mi355x, v.topk_ids, np.int32, T * k, stream).reshape(T, k),
            "w": read_device(mi355x, v.topk_w, np.float32, T * k, stream).reshape(T, k),
            "shared_w": read_device(mi355x, v.shared_w, np.float32, T, stream),
            "counts": read_device(mi355x, v.counts, np.int32, E, stream),
            "offsets": read_device(mi355x, v.offsets, np.int32, E + 1, stream),
            "sorted_tok": read_device(mi355x, v.sorted_tok, np.int32, R, stream),
            "pair_pos": read_device(mi355x, v.pair_pos, np.int32, T * k, stream).reshape(T, k),
            "n_groups": int(read_device(mi355x, v.n_groups, np.int32, 1, stream)[0]),
            "n_mtiles": int(read_device(mi355x, v.n_mtiles, np.int32, 1, stream)[0]),
            "m_blk": v.m_blk,
        }
        return out, views
    finally:
        dl.close()


def check_routing(views, ref, logits, bias, spec, label, x=None, t=None):
    """Whole-batch routing parity (tests/_routing.py rules): ids on every clear token,
    ties exchanged only among near-tied candidates, weights at the device ids, and every
    integer dispatch table bit for bit.  When the device exchanged tied experts and
    (x, t) are given, ``ref`` is re-evaluated on the device's selection in place."""
    T, k = ref["ids"].shape
    d = check_routing_tables(views, logits, bias, spec, len(views["counts"]), label,
                             has_shared=len(views["sorted_tok"]) > T * k)
    if x is not None and not np.array_equal(views["ids"], ref["ids"]):
        ref.update(orc.moe_block(x, t, spec, ids=views["ids"]))
    return d


# ---- golden vectors of the reference ----------------------------------------------------

@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_golden_on_gpu(mi355x, stream, name):
    say(f"[gpu] golden {name}")
    shape, x, t, ref_out = golden_case(name)
    spec = spec_for(shape)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    check_routing(views, ref, ref["logits"], t.get("mlp.gate.e_score_correction_bias"), spec, name,
                  x, t)
    if t["mlp.gate.weight"].dtype == np.float32:
        assert normwise_err(out, ref_out) <= FP32_REL, name
        assert normwise_err(out - x, ref_out - x) <= FP32_REL * 10, name
    else:
        assert float(np.max(np.abs(out - ref_out))) <= LOWP_ABS, name


# ---- router modes at config-1 shape (fp32) ----------------------------------------------

@pytest.mark.parametrize("mode", [orc.REF_SOFTMAX_BIAS, orc.SIGMOID_SELECT_BIAS, orc.SOFTMAX])
def test_router_modes_c1(mi355x, stream, mode):
    say(f"[gpu] c1 mode={mode}")
    shape = syn.C1
    t = syn.make_tensors(shape, 1234)
    x = syn.make_inputs(1234, 8, shape.hidden)
    spec = spec_for(shape, mode)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    check_routing(views, ref, ref["logits"], t["mlp.gate.e_score_correction_bias"], spec, mode,
                  x, t)
    assert normwise_err(out, ref["out"]) <= FP32_REL
    assert normwise_err(out - x, ref["out"] - x) <= FP32_REL * 10
    assert views["n_groups"] == 1 + len(np.unique(ref["ids"]))


# ---- token-count sweep: m-tile sizes 16/32/64 and multi-tile groups -----------------------

SWEEP_SHAPE = syn.MoeShape(syn.GLM, 256, 8, 3, 128, 64, 2.5, 1e-5)


@pytest.mark.parametrize("wdt", ["float32", "float16", "int8"])
@pytest.mark.parametrize("T", [1, 2, 5, 16, 17, 32, 33, 64, 100, 257])
def test_token_sweep(mi355x, stream, wdt, T):
    say(f"[gpu] sweep wdt={wdt} T={T}")
    shape = SWEEP_SHAPE
    base = syn.make_tensors(shape, 7 + T, norm_noise=0.1)
    if wdt == "float16":
        t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
                 else v) for n, v in base.items()}
    elif wdt == "int8":
        t = quantize_moe_tensors(base)
    else:
        t = base
    x = syn.make_inputs(7 + T, T, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)  # fp32 evaluation with the same (dequantised) weights
    check_routing(views, ref, ref["logits"], t["mlp.gate.e_score_correction_bias"], spec,
                  f"{wdt}/T={T}", x, t)
    if wdt == "float32":
        assert normwise_err(out, ref["out"]) <= FP32_REL
    else:
        err = float(np.max(np.abs(out - ref["out"])))
        say(f"    max abs err {err:.3e}")
        assert err <= LOWP_ABS


@pytest.mark.parametrize("wdt", ["float16", "int8"])
@pytest.mark.parametrize("T", [600, 1500])
def test_skewed_prefill(mi355x, stream, wdt, T):
    """Hot experts far above 128 rows (several m-tiles per group) next to cold ones."""
    say(f"[gpu] skewed prefill wdt={wdt} T={T}")
    shape = syn.MoeShape(syn.GLM, 512, 24, 4, 256, 128, 2.5, 1e-5)
    base = syn.make_tensors(shape, 99 + T)
    bias = np.zeros(shape.n_experts, np.float32)
    bias[:3] = [0.9, 0.5, 0.3]  # experts 0..2 take most tokens in sigmoid-select routing
    base["mlp.gate.e_score_correction_bias"] = bias
    if wdt == "float16":
        t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
                 else v) for n, v in base.items()}
    else:
        t = quantize_moe_tensors(base)
    x = syn.make_inputs(99 + T, T, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    assert ref["counts"][:3].min() > 256
    check_routing(views, ref, ref["logits"], bias, spec, f"skew/{wdt}/T={T}", x, t)
    err = float(np.max(np.abs(out - ref["out"])))
    say(f"    max abs err {err:.3e}, counts[:3]={ref['counts'][:3].tolist()}")
    assert err <= LOWP_ABS


@pytest.mark.parametrize("H,inter,shared,frag", [
    (768, 200, 136, False),    # 4-wave chains of 2 and 1 slabs, partial last stages
    (768, 192, 128, True),
    (1536, 1024, 512, True),   # 8-wave chains of 2 and 1 slabs
])
def test_prefill_slab_chains(mi355x, stream, H, inter, shared, frag):
    """fp16 prefill down projections run as slab chains (a block takes two column slabs of
    its m-tile in turn, the next slab's loads in flight across the epilogue): odd slab
    counts give chains of two slabs and of one, short reductions end in partial stages,
    hot experts span several m-tiles."""
    say(f"[gpu] prefill slab chains H={H} inter={inter} shared={shared} frag16={frag}")
    shape = syn.MoeShape(syn.GLM, H, 24, 4, inter, shared, 2.5, 1e-5)
    base = syn.make_tensors(shape, 4343)
    bias = np.zeros(shape.n_experts, np.float32)
    bias[:3] = [0.8, 0.4, 0.2]
    base["mlp.gate.e_score_correction_bias"] = bias
    t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
             else v) for n, v in base.items()}
    x = syn.make_inputs(4343, 700, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    out, views = run_device(mi355x, stream, t, shape, spec, x, frag=frag)
    ref = orc.moe_block(x, t, spec)
    assert views["m_blk"] == 128 and ref["counts"][:3].min() > 128
    check_routing(views, ref, ref["logits"], bias, spec, f"slab chains/{frag}", x, t)
    err = float(np.max(np.abs(out - ref["out"])))
    say(f"    max abs err {err:.3e}, counts[:3]={ref['counts'][:3].tolist()}")
    assert err <= LOWP_ABS


def test_prefill_eight_wave_blocks(mi355x, stream):
    """fp16 reductions of 1024-3072 columns run the prefill kernel with 8-wave blocks (gate/up
    over hidden 1024, down over inter 1024); the shared expert is narrower (320 columns), so
    some waves of its blocks own no columns, and two hot experts span several m-tiles."""
    say("[gpu] 8-wave prefill blocks")
    shape = syn.MoeShape(syn.GLM, 1024, 16, 4, 1024, 320, 2.5, 1e-5)
    base = syn.make_tensors(shape, 4242)
    bias = np.zeros(shape.n_experts, np.float32)
    bias[:2] = [0.6, 0.3]
    base["mlp.gate.e_score_correction_bias"] = bias
    t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
             else v) for n, v in base.items()}
    x = syn.make_inputs(4242, 300, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    assert views["m_blk"] == 128 and ref["counts"][:2].min() > 128
    check_routing(views, ref, ref["logits"], bias, spec, "eight-wave", x, t)
    err = float(np.max(np.abs(out - ref["out"])))
    say(f"    max abs err {err:.3e}, counts[:2]={ref['counts'][:2].tolist()}")
    assert err <= LOWP_ABS


# ---- Qwen3-Next structure: softmax router, no bias, gated shared expert --------------------

@pytest.mark.parametrize("wdt", ["float32", "float16"])
def test_qwen_structure(mi355x, stream, wdt):
    say(f"[gpu] qwen wdt={wdt}")
    shape = syn.MoeShape(syn.QWEN, 512, 64, 10, 128, 96, 1.0, 1e-6, has_bias=False,
                         has_shared_gate=True)
    t = syn.make_tensors(shape, 21, weight_dtype=np.dtype(wdt))
    x = syn.make_inputs(21, 40, shape.hidden)
    spec = spec_for(shape)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    check_routing(views, ref, ref["logits"], None, spec, f"qwen/{wdt}", x, t)
    np.testing.assert_allclose(views["shared_w"], ref["shared_w"], rtol=1e-5)
    if wdt == "float32":
        assert normwise_err(out, ref["out"]) <= FP32_REL
    else:
        assert float(np.max(np.abs(out - ref["out"]))) <= LOWP_ABS


# ---- many experts, 1-2 tokens: the top-k spread over several waves per token ---------------

@pytest.mark.parametrize("E,k,mode,T", [(512, 10, orc.SOFTMAX, 1), (512, 10, orc.SOFTMAX, 2),
                                        (400, 8, orc.SIGMOID_SELECT_BIAS, 1),
                                        (512, 32, orc.REF_SOFTMAX_BIAS, 2),
                                        (384, 6, orc.SOFTMAX, 2)])
def test_many_experts_small_batch(mi355x, stream, E, k, mode, T):
    say(f"[gpu] many experts E={E} k={k} mode={mode} T={T}")
    qwen = mode == orc.SOFTMAX
    shape = syn.MoeShape(syn.QWEN if qwen else syn.GLM, 256, E, k, 64, 64,
                         1.0 if qwen else 2.5, 1e-6, has_bias=not qwen, has_shared_gate=qwen)
    t = syn.make_tensors(shape, 77 + E + k)
    x = syn.make_inputs(77 + T, T, shape.hidden)
    spec = spec_for(shape, mode)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    check_routing(views, ref, ref["logits"], t.get("mlp.gate.e_score_correction_bias"), spec,
                  f"E{E}/k{k}/{mode}/T{T}", x, t)
    if qwen:
        np.testing.assert_allclose(views["shared_w"], ref["shared_w"], rtol=1e-5)
    assert normwise_err(out, ref["out"]) <= FP32_REL


def test_many_experts_ties_match_single_wave_selection(mi355x, stream):
    """Exact key ties (router rows repeated in groups of 4) go to the lower expert id on both
    selection paths: one token (several waves per token) against the same token repeated
    eight times (one wave per token)."""
    say("[gpu] many experts, tied keys")
    shape = syn.MoeShape(syn.QWEN, 256, 512, 10, 64, 64, 1.0, 1e-6, has_bias=False,
                         has_shared_gate=True)
    t = syn.make_tensors(shape, 5)
    w = t["mlp.gate.weight"]
    t["mlp.gate.weight"] = np.ascontiguousarray(np.repeat(w[::4], 4, axis=0))
    spec = spec_for(shape)
    x1 = syn.make_inputs(9, 1, shape.hidden)
    _, v1 = run_device(mi355x, stream, t, shape, spec, x1)
    _, v8 = run_device(mi355x, stream, t, shape, spec, np.repeat(x1, 8, axis=0))
    ids1 = v1["ids"][0]
    assert np.all(ids1 % 4 == 0) or len(set(ids1 // 4)) < len(ids1), "no tied group selected"
    for r in range(8):
        assert np.array_equal(v8["ids"][r], ids1), f"row {r}: {v8['ids'][r]} vs {ids1}"
        np.testing.assert_allclose(v8["w"][r], v1["w"][0], rtol=1e-6, atol=1e-7)


# ---- one token: the experts are selected inside the gate/up launch ------------------------

@pytest.mark.parametrize("E,k,mode,shared", [
    (512, 32, orc.REF_SOFTMAX_BIAS, True),    # 4 waves x 128 experts, 128 candidates
    (300, 32, orc.SIGMOID_SELECT_BIAS, True),
    (257, 4, orc.SIGMOID_SELECT_BIAS, False),  # first size past one wave's 256 experts
    (256, 16, orc.SOFTMAX, True),              # one wave, 4 experts per lane
    (9, 8, orc.REF_SOFTMAX_BIAS, False),       # one expert more than top-k
])
def test_one_token_selection_edges(mi355x, stream, E, k, mode, shared):
    say(f"[gpu] one token E={E} k={k} mode={mode} shared={shared}")
    qwen = mode == orc.SOFTMAX
    shape = syn.MoeShape(syn.QWEN if qwen else syn.GLM, 256, E, k, 64, 64 if shared else 0,
                         1.0 if qwen else 2.5, 1e-6, has_bias=not qwen,
                         has_shared_gate=qwen and shared)
    t = syn.make_tensors(shape, 300 + E + k)
    x = syn.make_inputs(301 + E, 1, shape.hidden)
    spec = spec_for(shape, mode)
    out, views = run_device(mi355x, stream, t, shape, spec, x)
    ref = orc.moe_block(x, t, spec)
    check_routing(views, ref, ref["logits"], t.get("mlp.gate.e_score_correction_bias"), spec,
                  f"one token E{E}/k{k}/{mode}", x, t)
    assert views["n_groups"] == k + (1 if shared else 0)
    assert views["n_mtiles"] == k + (1 if shared else 0)
    assert normwise_err(out, ref["out"]) <= FP32_REL


@pytest.mark.parametrize("E,k,mode", [(160, 8, orc.SIGMOID_SELECT_BIAS),
                                      (512, 10, orc.SOFTMAX)])
def test_one_token_split_stages_match_one_call(mi355x, stream, E, k, mode):
    """The staged entry (stages 0-3, then 4-6, as the expert-granular runtime calls it) keeps
    the top-k/dispatch launch; one call selects inside the gate/up launch.  Same ids and
    dispatch tables, outputs equal to fp32 rounding."""
    say(f"[gpu] one token, staged vs one call, E={E}")
    qwen = mode == orc.SOFTMAX
    shape = syn.MoeShape(syn.QWEN if qwen else syn.GLM, 256, E, k, 64, 64,
                         1.0 if qwen else 2.5, 1e-6, has_bias=not qwen, has_shared_gate=qwen)
    t = syn.make_tensors(shape, 400 + E)
    x = syn.make_inputs(401 + E, 1, shape.hidden)
    spec = spec_for(shape, mode)
    dl = DeviceMoeLayer.from_host(mi355x, t, stream)
    try:
        cfg = dl.config(top_k=k, router_mode=MODE_CODE[mode], routed_scaling=spec.routed_scaling,
                        eps=spec.eps, norm_topk_prob=spec.norm_topk_prob)
        desc = cfg.desc()

        def tables():
            v = dl.runner.views(desc, 1)
            return [read_device(mi355x, p, np.int32, n, stream) for p, n in
                    ((v.topk_ids, k), (v.sorted_tok, k + 1), (v.pair_pos, k),
                     (v.g_expert, k + 1), (v.g_start, k + 1), (v.mt_group, k + 1))]

        one = dl.forward_numpy(cfg, x)
        t_one = tables()
        w = dl.prepare(cfg, 1)
        used = dl.runner.route_numpy(desc, w, x, stream)
        staged = dl.runner.finish_numpy(desc, w, stream)
        t_staged = tables()
    finally:
        dl.close()
    assert used == sorted(int(e) for e in t_one[0])
    for a, b in zip(t_one, t_staged):
        assert np.array_equal(a, b)
    np.testing.assert_allclose(staged, one, rtol=1e-5, atol=1e-6)


# ---- error paths through the ABI ----------------------------------------------------------

def test_forward_rejects_bad_arguments(mi355x, stream):
    say("[gpu] error paths")
    lib = _lib.load()
    desc = _lib.MxMoeDesc(hidden=64, inter=32, shared_inter=0, n_experts=4, top_k=5,
                          router_mode=0, norm_topk_prob=1, weight_dtype=_lib.MX_DT_F32,
                          param_dtype=_lib.MX_DT_F32, has_bias=0, has_shared_gate=0,
                          routed_scaling=1.0, eps=1e-5)
    n = ctypes.c_size_t()
    assert lib.mx_moe_workspace_size(ctypes.byref(desc), 4, ctypes.byref(n)) == _lib.MX_ERR_INVALID
    desc.top_k = 2
    assert lib.mx_moe_workspace_size(ctypes.byref(desc), 4, ctypes.byref(n)) == _lib.MX_OK
    w = _lib.MxMoeWeights()
    rc = lib.mx_moe_forward(ctypes.byref(desc), ctypes.byref(w), None, None, 4, None, 0, stream)
    assert rc == _lib.MX_ERR_INVALID
    ws = mi355x.alloc_device(64)
    x = mi355x.alloc_device(4 * 64 * 4)
    try:
        w.norm_w = w.router_w = w.experts = x.handle
        rc = lib.mx_moe_forward(ctypes.byref(desc), ctypes.byref(w), x.handle, x.handle, 4,
                                ws.handle, 64, stream)
        assert rc == _lib.MX_ERR_WORKSPACE
    finally:
        mi355x.free_device(ws)
        mi355x.free_device(x)


def test_zero_tokens_is_a_no_op(mi355x, stream):
    say("[gpu] zero tokens")
    shape = syn.MoeShape(syn.GLM, 64, 4, 2, 32, 32, 2.5, 1e-5)
    t = syn.make_tensors(shape, 3)
    dl = DeviceMoeLayer.from_host(mi355x, t, stream)
    try:
        cfg = dl.config(top_k=2, router_mode=0, routed_scaling=2.5, eps=1e-5)
        out = dl.forward_numpy(cfg, np.zeros((0, 64), np.float32))
        assert out.shape == (0, 64)
    finally:
        dl.close()


# ---- dispatch: chunked (many workgroups) == single workgroup ---------------------------

@pytest.mark.parametrize("T,k,E,m_blk", [(1000, 8, 160, 128), (4096, 10, 512, 128),
                                         (300, 4, 24, 64), (257, 3, 8, 32)])
def test_chunked_dispatch_matches_single_workgroup(mi355x, stream, T, k, E, m_blk):
    say(f"[gpu] dispatch T={T} k={k} E={E}")
    lib = _lib.load()
    rng = np.random.default_rng(T + E)
    # skewed expert popularity, distinct ids per token
    p = rng.zipf(1.3, size=E * 4).astype(np.float64)[:E]
    p = p / p.sum()
    ids = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    tw = rng.random((T, k)).astype(np.float32)
    shw = rng.random(T).astype(np.float32)
    P = T * k
    R = P + T
    mtmax = P // m_blk + min(P, E) + (T + m_blk - 1) // m_blk
    sizes = {"counts": E, "offsets": E + 1, "sorted_tok": R, "sorted_w": R, "pair_pos": P,
             "g_expert": E + 1, "g_start": E + 1, "g_count": E + 1, "n_groups": 1,
             "mt_group": mtmax, "mt_row0": mtmax, "n_mtiles": 1}
    n = ctypes.c_size_t()
    assert lib.mx_dispatch_scratch_size(T, k, E, ctypes.byref(n)) == 0
    bufs = []

    def dev(nbytes):
        b = mi355x.alloc_device(max(nbytes, 16))
        bufs.append(b)
        return b.handle

    try:
        d_ids, d_tw, d_sw = dev(ids.nbytes), dev(tw.nbytes), dev(shw.nbytes)
        for h, a in ((d_ids, ids), (d_tw, tw), (d_sw, shw)):
            mi355x.copy_h2d_ptr_async(h, a.ctypes.data, a.nbytes, stream)
        scratch = dev(n.value)
        outs = {}
        for variant in ("single", "chunked"):
            o = {name: dev(cnt * 4) for name, cnt in sizes.items()}
            args = [o[name] for name in sizes]
            if variant == "single":
                rc = lib.mx_dispatch(d_ids, d_tw, d_sw, T, k, E, 1, m_blk, *args, stream)
            else:
                rc = lib.mx_dispatch_chunked(d_ids, d_tw, d_sw, T, k, E, 1, m_blk, scratch, *args,
                                             stream)
            assert rc == 0
            mi355x.synchronize_stream(stream)
            outs[variant] = {name: read_device(mi355x, o[name],
                                               np.float32 if name == "sorted_w" else np.int32,
                                               cnt, stream) for name, cnt in sizes.items()}
        a, b = outs["single"], outs["chunked"]
        ng, nm = int(a["n_groups"][0]), int(a["n_mtiles"][0])
        assert ng == int(b["n_groups"][0]) and nm == int(b["n_mtiles"][0])
        for name in ("counts", "offsets", "sorted_tok", "sorted_w", "pair_pos"):
            assert np.array_equal(a[name], b[name]), name
        for name in ("g_expert", "g_start", "g_count"):
            assert np.array_equal(a[name][:ng], b[name][:ng]), name
        for name in ("mt_group", "mt_row0"):
            assert np.array_equal(a[name][:nm], b[name][:nm]), name
        ref = orc.dispatch(ids, E)
        assert np.array_equal(a["counts"], ref["counts"])
        assert np.array_equal(a["sorted_tok"][:P], ref["sorted_tok"])
        assert np.array_equal(a["pair_pos"].reshape(T, k), ref["pair_pos"])
    finally:
        for b in bufs:
            mi355x.free_device(b)
