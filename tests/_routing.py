"""Whole-batch routing parity: device selection and dispatch tables against the oracle.

Rules (applied to every token of the batch):
  * a token whose k + 1 largest fp64 selection keys are all more than ``margin`` apart
    ("clear") must select exactly the oracle's ids, in the oracle's slot order;
  * on a near-tied token the device may only exchange near-tied candidates: its ids are
    distinct, and the key of its j-th id lies within ``margin`` of the j-th largest key;
  * the routing weights must equal the oracle's weights *at the device's ids*;
  * the integer dispatch tables (per-expert counts, offsets, the expert-sorted token
    order, the inverse permutation, the shared rows) are compared bit for bit with the
    oracle's dispatch of the device's ids.  On clear tokens those ids are the oracle's
    own, so every table is always compared, near ties or not.
"""
from __future__ import annotations

import sys

import numpy as np

from oracle import moe_oracle as orc

MARGIN = 1e-5


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def tie_ok(dev_ids: np.ndarray, keys: np.ndarray, margin: float) -> np.ndarray:
    """Per token: the device's ids are distinct and each lies within ``margin`` of the
    key rank it occupies (so it differs from the exact selection only among ties)."""
    T, k = dev_ids.shape
    s = -np.sort(-keys, axis=-1)[:, :k]
    got = np.take_along_axis(keys, dev_ids.astype(np.int64), axis=-1)
    distinct = np.array([len(set(r.tolist())) == k for r in dev_ids])
    return distinct & np.all(np.abs(got - s) <= margin, axis=-1)


def check_routing_tables(dev: dict, logits: np.ndarray, bias, spec: orc.MoeSpec, n_exp: int,
                         label: str, has_shared: bool = False, margin: float = MARGIN,
                         max_near_frac: float = 0.1) -> dict:
    """Compare the device routing of a whole batch with the oracle (rules above).

    ``dev`` holds the device's ``ids`` [T, k], ``w`` [T, k], ``counts`` [E],
    ``offsets`` [E + 1], ``sorted_tok`` [T k (+ T)] and ``pair_pos`` [T, k].  Returns the
    oracle's dispatch of the device ids (with ``near``: the near-tied token indices)."""
    ids = np.asarray(dev["ids"]).astype(np.int64)
    T, k = ids.shape
    if T == 0:
        return {"near": np.zeros(0, np.int64)}
    assert ids.min() >= 0 and ids.max() < n_exp, f"{label}: expert id out of range"
    ref_ids, _ = orc.route(logits, bias, spec)
    clear = orc.order_margin(logits, bias, spec) > margin
    near = np.flatnonzero(~clear)
    if near.size:
        say(f"{label}: {near.size} of {T} tokens near-tied (key gap <= {margin}): "
            f"{near[:32].tolist()}{' ...' if near.size > 32 else ''}")
    assert near.size <= max(1, max_near_frac * T), f"{label}: too many near-tied tokens"
    bad = np.flatnonzero(clear & np.any(ids != ref_ids, axis=-1))
    assert bad.size == 0, (f"{label}: expert ids differ from the oracle on clear tokens "
                           f"{bad[:16].tolist()}: device {ids[bad[:4]].tolist()} oracle "
                           f"{ref_ids[bad[:4]].tolist()}")
    if near.size:
        keys = orc.selection_keys(logits, bias, spec)
        ok = tie_ok(ids[near], keys[near], margin)
        assert ok.all(), (f"{label}: near-tied tokens {near[~ok][:16].tolist()} select "
                          "beyond the tie")
        swapped = near[np.any(ids[near] != ref_ids[near], axis=-1)]
        if swapped.size:
            say(f"{label}: tokens {swapped[:16].tolist()} exchanged near-tied experts")
    w_ref = orc.route_weights(logits, bias, ids, spec)
    np.testing.assert_allclose(np.asarray(dev["w"]), w_ref, rtol=1e-5, atol=1e-6,
                               err_msg=f"{label}: routing weights")
    ref = orc.dispatch(ids.astype(np.int32), n_exp)
    assert np.array_equal(np.asarray(dev["counts"]), ref["counts"]), f"{label}: counts"
    assert np.array_equal(np.asarray(dev["offsets"]), ref["offsets"]), f"{label}: offsets"
    st = np.asarray(dev["sorted_tok"])
    assert np.array_equal(st[: T * k], ref["sorted_tok"]), f"{label}: expert-sorted order"
    assert np.array_equal(np.asarray(dev["pair_pos"]).reshape(T, k), ref["pair_pos"]), \
        f"{label}: inverse permutation"
    if has_shared:
        assert np.array_equal(st[T * k: T * k + T], np.arange(T)), f"{label}: shared rows"
    ref["near"] = near
    return ref
