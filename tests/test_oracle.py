"""Pin the CPU oracle: reference golden vectors, the reference's own KATs, closed forms,
brute force on tiny inputs, and invariants chosen so that a dropped term, a wrong sign or
a swapped operand fails."""
from __future__ import annotations

import itertools

import numpy as np
import pytest

from _cases import golden_case, golden_cases, normwise_err, spec_for
from moe_mi355x import synthetic as syn
from oracle import moe_oracle as orc


# ---- golden vectors written by the reference executors --------------------------------

@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_faithful_matches_reference_golden(name):
    shape, x, t, ref = golden_case(name)
    out = orc.moe_block_faithful(x, t, spec_for(shape))
    # Same NumPy operations in the same order: agreement to the last few ulps.
    assert normwise_err(out, ref) < 1e-6


@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_grouped_matches_reference_golden(name):
    shape, x, t, ref = golden_case(name)
    res = orc.moe_block(x, t, spec_for(shape))
    assert normwise_err(res["out"], ref) < 1e-5
    assert normwise_err(res["out"] - x, ref - x) < 1e-5


def test_golden_detects_a_wrong_router():
    """A plausible mistake — bias applied after the softmax — must miss the golden."""
    shape, x, t, ref = golden_case("glm_c1_f32")
    spec = spec_for(shape)
    h = orc.rms_norm(x, t["post_attention_layernorm.weight"], spec.eps)
    logits = orc.router_logits(h, t)
    b = t["mlp.gate.e_score_correction_bias"]
    p = orc.softmax(logits) + b  # wrong order
    ids = np.argsort(-p, axis=-1)[:, : spec.top_k]
    good_ids, _ = orc.route(logits, b, spec)
    assert not np.array_equal(np.sort(ids, axis=1), np.sort(good_ids, axis=1)) or \
        normwise_err(orc.moe_block_faithful(x, t, orc.MoeSpec(spec.top_k, orc.SOFTMAX, True,
                                                               spec.routed_scaling, spec.eps)),
                     ref) > 1e-4


def test_golden_detects_missing_scaling():
    shape, x, t, ref = golden_case("glm_c1_f32")
    spec = spec_for(shape)
    wrong = orc.MoeSpec(spec.top_k, spec.router_mode, True, 1.0, spec.eps)
    assert normwise_err(orc.moe_block_faithful(x, t, wrong) - x, ref - x) > 1e-2


# ---- the reference's own KATs (tests/test_executor_np.py:151-202) ----------------------

def test_primitive_kats():
    np.testing.assert_allclose(orc.rms_norm(np.ones((1, 4), np.float32), np.ones(4, np.float32)),
                               1.0, atol=1e-5)
    np.testing.assert_allclose(orc.rms_norm(np.full((1, 2), 2.0, np.float32),
                                            np.ones(2, np.float32)), 1.0, atol=1e-5)
    assert abs(float(orc.silu(np.array(0.0)))) < 1e-6
    assert float(orc.silu(np.array(5.0))) > 4.9
    s = orc.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    np.testing.assert_allclose(s.sum(), 1.0, atol=1e-6)
    assert int(np.argmax(orc.softmax(np.array([1.0, 10.0, 2.0], np.float32)))) == 1
    np.testing.assert_allclose(orc.linear_t(np.array([[1.0, 0.0]], np.float32),
                                            np.array([[2.0, 3.0]], np.float32)), [[2.0]])


def test_primitive_closed_forms():
    x = np.array([[3.0, -4.0]], np.float32)  # mean(x^2) = 12.5
    w = np.array([2.0, 0.5], np.float32)
    np.testing.assert_allclose(orc.rms_norm(x, w, eps=0.0), w * x / np.sqrt(12.5), rtol=1e-6)
    v = np.linspace(-8, 8, 33)
    np.testing.assert_allclose(orc.silu(v), v / (1 + np.exp(-v)), rtol=1e-12)
    np.testing.assert_allclose(orc.sigmoid(np.array([0.0, np.log(3.0)])), [0.5, 0.75], rtol=1e-12)


# ---- int8 (reference KATs tests/test_quantize.py:41-54) and the per-row scheme ---------

def test_dequant_kats():
    np.testing.assert_allclose(orc.dequant_int8_layer(bytes([4, 0xFE]), 0.5, 0), [2.0, -1.0])
    np.testing.assert_allclose(orc.dequant_int8_layer(bytes([15]), 1.0, 10), [5.0])
    np.testing.assert_allclose(orc.dequant_int8_layer(bytes([3, 0xFF]), 2.0), [6.0, -2.0])


def test_quantize_rows_known_values():
    w = np.array([[0.5, -1.27, 0.0], [0.0, 0.0, 0.0], [127.0, 2.5, -2.5]], np.float32)
    q, s = orc.quantize_rows_int8(w)
    assert s.dtype == np.float16
    assert s[0] == np.float16(0.01) and s[1] == 1.0 and s[2] == 1.0
    assert q[0].tolist() == [50, -127, 0]
    assert q[1].tolist() == [0, 0, 0]
    assert q[2].tolist() == [127, 2, -2]  # round half to even


def test_quantize_rows_error_bound_and_package_agree():
    from moe_mi355x.quantize import dequantize_rows_int8, quantize_rows_int8

    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    q, s = orc.quantize_rows_int8(w)
    q2, s2 = quantize_rows_int8(w)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint16), s2.view(np.uint16))
    deq = dequantize_rows_int8(q, s)
    # |W - W'| <= scale/2 (+ the fp16 rounding of the scale itself)
    bound = s.astype(np.float32)[:, None] * 0.5 + np.abs(w) * 2 ** -10
    assert np.all(np.abs(deq - w) <= bound + 1e-9)


# ---- router: brute force in fp64 on tiny inputs -----------------------------------------

def _brute_route(logits, bias, spec):
    l64 = logits.astype(np.float64)
    T, E = l64.shape
    ids = np.zeros((T, spec.top_k), np.int64)
    ws = np.zeros((T, spec.top_k), np.float64)
    for t in range(T):
        if spec.router_mode == orc.SIGMOID_SELECT_BIAS:
            score = 1.0 / (1.0 + np.exp(-l64[t]))
            key = score + bias.astype(np.float64)
        else:
            z = l64[t] + (bias.astype(np.float64) if spec.router_mode == orc.REF_SOFTMAX_BIAS
                          else 0.0)
            score = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
            key = z
        best = sorted(range(E), key=lambda e: (-key[e], e))[: spec.top_k]
        w = score[best]
        if spec.norm_topk_prob:
            w = w / w.sum()
        ids[t] = best
        ws[t] = w * spec.routed_scaling
    return ids, ws


@pytest.mark.parametrize("mode", [orc.REF_SOFTMAX_BIAS, orc.SIGMOID_SELECT_BIAS, orc.SOFTMAX])
@pytest.mark.parametrize("norm", [True, False])
def test_route_matches_brute_force(mode, norm):
    rng = np.random.default_rng(42)
    T, E, k = 6, 9, 3
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    spec = orc.MoeSpec(top_k=k, router_mode=mode, norm_topk_prob=norm, routed_scaling=2.5)
    ids, w = orc.route(logits, bias, spec)
    bids, bw = _brute_route(logits, bias, spec)
    assert np.array_equal(ids, bids)
    np.testing.assert_allclose(w, bw, rtol=2e-6)
    if norm:
        np.testing.assert_allclose(w.sum(axis=1), 2.5, rtol=1e-6)


def test_sigmoid_mode_hand_example():
    # keys: sigmoid(0) + 1 = 1.5 > sigmoid(2) = 0.88 > sigmoid(1) = 0.73
    logits = np.array([[0.0, 1.0, 2.0]], np.float32)
    bias = np.array([1.0, 0.0, 0.0], np.float32)
    spec = orc.MoeSpec(top_k=2, router_mode=orc.SIGMOID_SELECT_BIAS, norm_topk_prob=True,
                       routed_scaling=2.5)
    ids, w = orc.route(logits, bias, spec)
    assert ids.tolist() == [[0, 2]]
    s0, s2 = 0.5, 1 / (1 + np.exp(-2.0))  # weights come from the unbiased scores
    np.testing.assert_allclose(w, [[2.5 * s0 / (s0 + s2), 2.5 * s2 / (s0 + s2)]], rtol=1e-6)


def test_ref_mode_hand_example():
    # softmax(l + b): selection and weights both use the biased probabilities
    logits = np.array([[0.0, 1.0, 2.0]], np.float32)
    bias = np.array([3.0, 0.0, 0.0], np.float32)
    spec = orc.MoeSpec(top_k=1, router_mode=orc.REF_SOFTMAX_BIAS, norm_topk_prob=False,
                       routed_scaling=1.0)
    ids, w = orc.route(logits, bias, spec)
    z = np.array([3.0, 1.0, 2.0])
    assert ids.tolist() == [[0]]
    np.testing.assert_allclose(w, [[np.exp(3) / np.exp(z).sum()]], rtol=1e-6)


# ---- dispatch invariants and brute force ------------------------------------------------

def test_dispatch_matches_token_mask_order():
    rng = np.random.default_rng(5)
    T, E, k = 37, 11, 4
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    d = orc.dispatch(ids, E)
    assert d["counts"].sum() == T * k
    # brute force: the rows expert e gathers with h[token_mask], in order
    rows = []
    for e in range(E):
        token_mask = (ids == e).any(axis=-1)
        rows += np.where(token_mask)[0].tolist()
    assert d["sorted_tok"].tolist() == rows
    # pair_pos is a permutation, and row pair_pos[t, j] belongs to expert ids[t, j]
    pp = d["pair_pos"]
    assert sorted(pp.ravel().tolist()) == list(range(T * k))
    row_expert = np.repeat(np.arange(E), d["counts"])
    assert np.array_equal(row_expert[pp], ids)
    assert np.array_equal(d["sorted_tok"][pp], np.repeat(np.arange(T)[:, None], k, axis=1))


# ---- expert products: fp64 brute force --------------------------------------------------

def test_swiglu_brute_force():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 5)).astype(np.float32)
    g, u = rng.standard_normal((2, 4, 5)).astype(np.float32)
    d = rng.standard_normal((5, 4)).astype(np.float32)
    out = orc.swiglu(x, g, u, d)
    ref = np.zeros((3, 5))
    for t, o in itertools.product(range(3), range(5)):
        acc = 0.0
        for i in range(4):
            gv = sum(float(x[t, c]) * float(g[i, c]) for c in range(5))
            uv = sum(float(x[t, c]) * float(u[i, c]) for c in range(5))
            acc += gv / (1 + np.exp(-gv)) * uv * float(d[o, i])
        ref[t, o] = acc
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mode", [orc.REF_SOFTMAX_BIAS, orc.SIGMOID_SELECT_BIAS])
def test_grouped_equals_faithful(mode):
    shape = syn.MoeShape(syn.GLM, 64, 8, 3, 32, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 11)
    x = syn.make_inputs(11, 13, 64)
    spec = spec_for(shape, mode)
    a = orc.moe_block_faithful(x, t, spec)
    b = orc.moe_block(x, t, spec)["out"]
    assert normwise_err(b, a) < 1e-6


def test_block_brute_force_fp64():
    """The whole block on a tiny Qwen-style layer against a scalar fp64 evaluation."""
    shape = syn.MoeShape(syn.QWEN, 8, 5, 2, 4, 3, 1.0, 1e-6, has_bias=False, has_shared_gate=True)
    t = syn.make_tensors(shape, 2, norm_noise=0.3)
    x = syn.make_inputs(2, 4, 8)
    spec = spec_for(shape)
    out = orc.moe_block(x, t, spec)["out"]
    f = {k: v.astype(np.float64) for k, v in t.items()}
    for tok in range(4):
        xv = x[tok].astype(np.float64)
        h = f["post_attention_layernorm.weight"] * xv / np.sqrt(np.mean(xv ** 2) + 1e-6)
        lg = f["mlp.gate.weight"] @ h
        p = np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum()
        top = sorted(range(5), key=lambda e: -p[e])[:2]
        w = p[top] / p[top].sum()

        def sw(pre):
            gv = f[pre + "gate_proj.weight"] @ h
            uv = f[pre + "up_proj.weight"] @ h
            return f[pre + "down_proj.weight"] @ (gv / (1 + np.exp(-gv)) * uv)

        acc = sum(wj * sw(f"mlp.experts.{e}.") for wj, e in zip(w, top))
        gate = 1 / (1 + np.exp(-(f["mlp.shared_expert_gate.weight"] @ h)[0]))
        ref = xv + acc + gate * sw("mlp.shared_expert.")
        np.testing.assert_allclose(out[tok], ref, rtol=1e-5, atol=1e-6)


def test_int8_weights_are_dequantised():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 9)
    from moe_mi355x.quantize import quantize_moe_tensors

    tq = quantize_moe_tensors(t)
    w = orc.weight(tq, "mlp.experts.1.up_proj.weight")
    q, s = orc.quantize_rows_int8(t["mlp.experts.1.up_proj.weight"])
    np.testing.assert_array_equal(w, q.astype(np.float32) * s.astype(np.float32)[:, None])
