"""Router logit partials through the exported mx_router_logits against float64 products.

logits[s, t, e] summed over the slices s must equal h[t] . Wr[e] (e < E) and h[t] . w_sg
(e == E, the shared-expert gate row) -- glm4_moe.py:181, qwen3_next.py:278 and :328.
Long inputs with fp32 router rows run on the LDS-staged fp32 GEMM, the rest on the
direct-load router kernel; both are covered, with 1 to 16 slices, hidden sizes that are
and are not multiples of the slice granule, expert counts off the 128-column tile and the
shared gate row.

Tolerance: any fp32 evaluation of a K-term dot product in any order, with fp32 products,
is within K * 2**-24 * sum_k |h_k w_k| of the exact value (the worst-case bound of
recursive summation).  A slice left out, a wrong row or a transposed operand moves a
logit by about sqrt(K) * |h w|, far outside that bound at these sizes.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x.moe import read_device

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _slices_for(hidden: int, splits: int, gemm: bool) -> int:
    """The slice count the library accepts for `splits` (its slice granule is 16 columns
    on the GEMM path and 256 otherwise)."""
    g = 16 if gemm else 256
    kch = -(-hidden // g)
    per = -(-kch // splits)
    return -(-hidden // (per * g))


CASES = [
    # tokens, hidden, experts, shared gate, param dtype, splits, GEMM path expected
    (65, 256, 64, False, np.float32, 1, True),
    (300, 2048, 512, True, np.float32, 3, True),
    (1000, 5120, 160, False, np.float32, 16, True),
    (129, 1040, 130, True, np.float32, 5, True),
    (4100, 2048, 512, True, np.float32, 3, True),
    (200, 512, 64, True, np.float16, 2, False),
    (40, 768, 96, False, np.float32, 3, False),
]


@pytest.mark.parametrize("T,H,E,sg,pdt,splits,gemm", CASES)
def test_router_logits_match_float64(mi355x, stream, T, H, E, sg, pdt, splits, gemm):
    say(f"[gpu] router logits T={T} H={H} E={E} shared_gate={sg} {np.dtype(pdt).name} "
        f"splits={splits}")
    lib = _lib.load()
    rng = np.random.default_rng(T * 7 + H + E)
    h = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) * 0.05).astype(pdt)
    wsg = (rng.standard_normal((1, H)) * 0.05).astype(pdt) if sg else None
    e1 = E + (1 if sg else 0)
    S = _slices_for(H, splits, gemm)
    assert S == splits
    bufs = []
    try:
        def up(a):
            b = mi355x.alloc_device(a.nbytes)
            bufs.append(b)
            mi355x.copy_h2d_ptr_async(b.handle, a.ctypes.data, a.nbytes, stream)
            return b.handle
        dh, dw = up(h), up(w)
        dsg = up(wsg) if sg else None
        out = mi355x.alloc_device(S * T * e1 * 4)
        bufs.append(out)
        code = _lib.MX_DT_F32 if pdt == np.float32 else _lib.MX_DT_F16
        rc = lib.mx_router_logits(dh, dw, dsg, code, T, H, E, S, out.handle, stream)
        assert rc == 0, rc
        got = read_device(mi355x, out.handle, np.float32, S * T * e1, stream)
        # a slice count that does not match the granule is rejected
        if gemm and H // 16 >= 17:
            assert lib.mx_router_logits(dh, dw, dsg, code, T, H, E, H // 16 + 1, out.handle,
                                        stream) == _lib.MX_ERR_INVALID
    finally:
        mi355x.synchronize_stream(stream)
        for b in bufs:
            mi355x.free_device(b)
    got = got.reshape(S, T, e1).sum(axis=0, dtype=np.float64)
    rows = w.astype(np.float64) if not sg else np.concatenate(
        [w.astype(np.float64), wsg.astype(np.float64)])
    h64 = h.astype(np.float64)
    ref = h64 @ rows.T
    bound = H * 2.0 ** -24 * (np.abs(h64) @ np.abs(rows).T)
    err = np.abs(got - ref)
    assert np.all(err <= bound + 1e-30), (err.max(), (err / bound).max())
    # the sum of slices is not merely within the bound: typical errors are far smaller
    assert np.median(err / np.maximum(bound, 1e-30)) < 0.05


# The router inside the MoE block: for long inputs with fp16 / int8 expert weights it runs
# on the split-plane fp16 GEMM (h and the router rows as hi + 2^-11 lo planes).  Its logit
# partials are read back from the block's views and checked against float64 products of
# the RMSNorm output (evaluated in float64; the block's fp32 rows are within 2^-22 of it
# and are not kept on this path) with the router rows.  Each product is carried to
# within 3 * 2^-22 of its size (both planes rounded, the lo * lo term dropped), so the
# bound is (K + 16) * 2^-24 * sum |h w|, plus 2^-30 * (sum |w| + sum |h|) for the entries
# of h and w below fp16's normal range (each carried to within 2^-36).
BLOCK_CASES = [
    # shape (hidden, experts, top-k, inter, shared), shared gate, param dtype, tokens
    ((2048, 64, 4, 64, 64), True, np.float32, 300),
    ((1024, 160, 8, 64, 64), False, np.float32, 129),
    ((512, 96, 6, 64, 0), False, np.float16, 1100),
    ((2048, 512, 10, 32, 32), True, np.float32, 4096),
]


@pytest.mark.parametrize("dims,sg,pdt,T", BLOCK_CASES)
def test_block_router_logits_split_planes(mi355x, stream, dims, sg, pdt, T):
    from moe_mi355x import synthetic as syn
    from moe_mi355x.device_layer import DeviceMoeLayer

    H, E, k, inter, shared = dims
    say(f"[gpu] block router logits H={H} E={E} shared_gate={sg} {np.dtype(pdt).name} T={T}")
    arch = syn.QWEN if sg else syn.GLM
    shape = syn.MoeShape(arch, H, E, k, inter, shared, 1.0, 1e-6, has_bias=not sg,
                         has_shared_gate=sg)
    t = syn.make_tensors(shape, 4242 + T, weight_dtype=np.float16, param_dtype=pdt,
                         norm_noise=0.5)
    x = syn.make_inputs(4243 + T, T, H)
    dl = DeviceMoeLayer.from_host(mi355x, t, stream)
    try:
        mode = _lib.MX_ROUTER_SOFTMAX if sg else _lib.MX_ROUTER_REF_SOFTMAX_BIAS
        cfg = dl.config(top_k=k, router_mode=mode, routed_scaling=1.0, eps=1e-6)
        out = dl.forward_numpy(cfg, x)
        assert np.all(np.isfinite(out))
        v = dl.runner.views(cfg.desc(), T)
        S, e1 = v.router_splits, E + (1 if sg else 0)
        got = read_device(mi355x, v.logits, np.float32, S * T * e1, stream).reshape(S, T, e1)
    finally:
        dl.close()
    rows = t["mlp.gate.weight"].astype(np.float64)
    if sg:
        rows = np.concatenate([rows, t["mlp.shared_expert_gate.weight"].astype(np.float64)])
    x64 = x.astype(np.float64)
    h64 = (t["post_attention_layernorm.weight"].astype(np.float64)
           * (x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6)))
    ref = h64 @ rows.T
    got = got.sum(axis=0, dtype=np.float64)
    bound = ((H + 16) * 2.0 ** -24 * (np.abs(h64) @ np.abs(rows).T)
             + 2.0 ** -30 * (np.abs(rows).sum(axis=1)[None, :] + np.abs(h64).sum(axis=1)[:, None]))
    err = np.abs(got - ref)
    assert np.all(err <= bound), (err.max(), (err / bound).max())
    assert np.median(err / bound) < 0.05
