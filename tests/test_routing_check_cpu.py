"""The whole-batch routing check (tests/_routing.py) and the oracle pieces it rests on,
on the CPU: it accepts the oracle's own routing, accepts exchanges of exactly tied
experts, and rejects planted mistakes (a different expert on a clear token, a swapped
slot order, a wrong count or sorted row)."""
from __future__ import annotations

import numpy as np
import pytest

from _routing import check_routing_tables, tie_ok
from oracle import moe_oracle as orc

MODES = [orc.REF_SOFTMAX_BIAS, orc.SIGMOID_SELECT_BIAS, orc.SOFTMAX]


def _case(mode, T=200, E=32, k=4, seed=0):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (0.01 * rng.standard_normal(E)).astype(np.float32) if mode != orc.SOFTMAX else None
    spec = orc.MoeSpec(top_k=k, router_mode=mode, norm_topk_prob=True,
                       routed_scaling=2.5 if mode != orc.SOFTMAX else 1.0)
    return logits, bias, spec


def _device_from(ids, logits, bias, spec, E, shared=True):
    """What a correct device would report for the selection ``ids``."""
    T, k = ids.shape
    d = orc.dispatch(ids.astype(np.int32), E)
    st = np.concatenate([d["sorted_tok"], np.arange(T, dtype=np.int32)]) if shared \
        else d["sorted_tok"]
    return {"ids": ids.astype(np.int32), "w": orc.route_weights(logits, bias, ids, spec),
            "counts": d["counts"], "offsets": d["offsets"], "sorted_tok": st,
            "pair_pos": d["pair_pos"]}


@pytest.mark.parametrize("mode", MODES)
def test_accepts_the_oracle_routing(mode):
    logits, bias, spec = _case(mode)
    ids, w = orc.route(logits, bias, spec)
    dev = _device_from(ids, logits, bias, spec, 32)
    np.testing.assert_array_equal(dev["w"], w)  # route_weights reproduces route's weights
    ref = check_routing_tables(dev, logits, bias, spec, 32, mode, has_shared=True)
    assert np.array_equal(ref["counts"], np.bincount(ids.ravel(), minlength=32))


@pytest.mark.parametrize("mode", MODES)
def test_rejects_a_different_expert_on_a_clear_token(mode):
    logits, bias, spec = _case(mode)
    ids, _ = orc.route(logits, bias, spec)
    t = int(np.flatnonzero(orc.order_margin(logits, bias, spec) > 1e-3)[0])
    bad = ids.copy()
    bad[t, -1] = next(e for e in range(32) if e not in ids[t])
    with pytest.raises(AssertionError, match="clear"):
        check_routing_tables(_device_from(bad, logits, bias, spec, 32), logits, bias, spec, 32,
                             mode, has_shared=True)


def test_rejects_a_swapped_slot_order():
    logits, bias, spec = _case(orc.SOFTMAX)
    ids, _ = orc.route(logits, bias, spec)
    t = int(np.flatnonzero(orc.order_margin(logits, bias, spec) > 1e-3)[0])
    bad = ids.copy()
    bad[t, [0, 1]] = bad[t, [1, 0]]
    with pytest.raises(AssertionError, match="clear"):
        check_routing_tables(_device_from(bad, logits, bias, spec, 32), logits, bias, spec, 32,
                             "order", has_shared=True)


@pytest.mark.parametrize("table", ["counts", "offsets", "sorted_tok", "pair_pos"])
def test_rejects_a_wrong_dispatch_table(table):
    logits, bias, spec = _case(orc.SIGMOID_SELECT_BIAS)
    ids, _ = orc.route(logits, bias, spec)
    dev = _device_from(ids, logits, bias, spec, 32)
    a = np.array(dev[table]).copy()
    flat = a.reshape(-1)
    if table == "counts":
        flat[[0, 1]] += [1, -1]
    else:
        flat[[3, 4]] = flat[[4, 3]] if flat[3] != flat[4] else flat[[3, 4]] + 1
    dev[table] = a
    with pytest.raises(AssertionError):
        check_routing_tables(dev, logits, bias, spec, 32, table, has_shared=True)


def test_rejects_wrong_weights():
    logits, bias, spec = _case(orc.REF_SOFTMAX_BIAS)
    ids, _ = orc.route(logits, bias, spec)
    dev = _device_from(ids, logits, bias, spec, 32)
    dev["w"] = dev["w"] * np.float32(1.001)
    with pytest.raises(AssertionError, match="weights"):
        check_routing_tables(dev, logits, bias, spec, 32, "w", has_shared=True)


@pytest.mark.parametrize("mode", MODES)
def test_accepts_an_exchange_of_exactly_tied_experts(mode):
    """Token 0's k-th and (k+1)-th keys are made equal; a device that picks the other one
    of the pair passes, and its tables are compared against the dispatch of its choice."""
    logits, bias, spec = _case(mode)
    k = spec.top_k
    keys = orc.selection_keys(logits, bias, spec)
    order = np.argsort(-keys[0])
    a, b = int(order[k - 1]), int(order[k])
    if bias is not None:
        bias = bias.copy()
        bias[b] = bias[a]
    logits[0, b] = logits[0, a]
    ids, _ = orc.route(logits, bias, spec)
    assert orc.order_margin(logits, bias, spec)[0] == 0.0
    alt = ids.copy()
    row = alt[0].tolist()
    other = b if a in row else a
    alt[0, row.index(a if a in row else b)] = other
    ref = check_routing_tables(_device_from(alt, logits, bias, spec, 32), logits, bias, spec,
                               32, mode, has_shared=True)
    assert 0 in ref["near"].tolist()
    np.testing.assert_allclose(orc.route_weights(logits, bias, alt, spec).sum(-1),
                               spec.routed_scaling, rtol=1e-6)


def test_tie_rule_brute_force():
    """tie_ok against a direct statement: distinct ids whose keys equal the sorted keys
    rank by rank within the margin."""
    rng = np.random.default_rng(3)
    keys = np.round(rng.standard_normal((300, 12)), 1)  # many exact ties
    k = 3
    for _ in range(5):
        ids = np.stack([rng.permutation(12)[:k] for _ in range(300)])
        ids[::2] = np.argsort(-keys[::2], kind="stable")[:, :k]
        got = tie_ok(ids, keys, 1e-9)
        for t in range(300):
            s = sorted(keys[t], reverse=True)
            want = len(set(ids[t])) == k and all(abs(keys[t][ids[t][j]] - s[j]) <= 1e-9
                                                 for j in range(k))
            assert got[t] == want


def test_order_margin_brute_force():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((50, 9)).astype(np.float32)
    spec = orc.MoeSpec(top_k=3, router_mode=orc.SOFTMAX)
    got = orc.order_margin(logits, None, spec)
    for t in range(50):
        s = sorted(logits[t].astype(np.float64), reverse=True)
        assert got[t] == min(s[j] - s[j + 1] for j in range(3))
