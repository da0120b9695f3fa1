"""The gated full-attention block on the GPU against the oracle
(oracle/full_attn_oracle.py, itself pinned to the reference's golden outputs)."""
from __future__ import annotations

import ctypes
import json
import sys

import numpy as np
import pytest

from _cases import GOLDEN, normwise_err
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.full_attn import DeviceFullAttnLayer
from moe_mi355x.moe import read_device
from moe_mi355x.quantize import quantize_rows_int8
from oracle import full_attn_oracle as fa

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def spec_of(s):
    return fa.FullAttnSpec(s.n_heads, s.n_kv_heads, s.head_dim, s.rotary_dim, s.rope_theta, s.eps)


def _layer(mi355x, stream, s, t):
    return DeviceFullAttnLayer.from_host(mi355x, t, s.n_heads, s.n_kv_heads, s.head_dim,
                                         s.rotary_dim, s.rope_theta, stream)


def _block(mi355x, stream, s, t, x, f16_act):
    layer = _layer(mi355x, stream, s, t)
    try:
        out = layer.forward_numpy(x, s.eps)
        T = x.shape[0]
        v = layer.runner.views(layer.desc(s.eps), T)
        nh, nkv, hd = s.n_heads, s.n_kv_heads, s.head_dim
        views = {
            "qg": read_device(mi355x, v.qg, np.float32, T * 2 * nh * hd, stream).reshape(T, -1),
            "k": read_device(mi355x, v.k, np.float32, T * nkv * hd, stream).reshape(T, -1),
            "v": read_device(mi355x, v.v, np.float32, T * nkv * hd, stream).reshape(T, -1),
            "act": read_device(mi355x, v.act, np.float16 if f16_act else np.float32,
                               T * nh * hd, stream).reshape(T, -1).astype(np.float32),
        }
        return out, views
    finally:
        layer.close()


def _golden():
    p = GOLDEN / "full_attn_index.json"
    return json.loads(p.read_text()) if p.exists() else {}


@pytest.mark.parametrize("name", sorted(_golden()))
def test_block_matches_reference_golden(mi355x, stream, name):
    case = _golden()[name]
    s = syn.FullAttnShape(**case["shape"])
    say(f"[gpu] full attention golden {name} {s}")
    dt = np.dtype(case["dtype"])
    t = syn.make_full_attn_tensors(s, case["seed"], weight_dtype=dt, param_dtype=dt,
                                   norm_noise=case["norm_noise"])
    x = syn.make_inputs(case["seed"], case["tokens"], s.hidden)
    out, _ = _block(mi355x, stream, s, t, x, dt == np.float16)
    want = np.load(GOLDEN / f"{name}.npz")["out"]
    err = float(np.max(np.abs(out - want)))
    say(f"    max abs err vs reference {err:.2e}")
    assert err <= (1e-4 if dt == np.float32 else 2e-2)


@pytest.mark.parametrize("hd,nh,nkv,wdt,T", [
    (16, 4, 2, "float32", 1), (64, 8, 2, "float32", 130), (128, 4, 1, "float32", 33),
    (256, 4, 2, "float32", 70), (64, 8, 4, "float16", 17), (256, 8, 2, "float16", 300),
    (128, 4, 2, "int8", 80), (32, 2, 2, "float16", 64)])
def test_block_intermediates_match_oracle(mi355x, stream, hd, nh, nkv, wdt, T):
    s = syn.FullAttnShape(256, nh, nkv, hd, 0.25, 5000000.0, 1e-6)
    say(f"[gpu] full attention hd={hd} heads={nh}/{nkv} {wdt} T={T}")
    t = syn.make_full_attn_tensors(s, 60 + T, weight_dtype=np.float16 if wdt == "int8"
                                   else np.dtype(wdt), norm_noise=0.1)
    ref_t = dict(t)
    if wdt == "int8":
        for k in (fa.Q, fa.K, fa.V, fa.O):
            q, sc = quantize_rows_int8(t[k].astype(np.float32))
            t[k], t[k + "_scale"] = q, sc
            ref_t[k] = q.astype(np.float32) * sc.astype(np.float32)[:, None]
    x = syn.make_inputs(70 + T, T, s.hidden)
    out, vw = _block(mi355x, stream, s, t, x, wdt != "float32")
    ref = fa.full_attn_block(x, ref_t, spec_of(s))
    exact = wdt == "float32"
    od = nh * hd
    q = ref["q"].transpose(1, 0, 2).reshape(T, od)
    k = ref["k"].transpose(1, 0, 2).reshape(T, nkv * hd)
    v = ref["v"].transpose(1, 0, 2).reshape(T, nkv * hd)
    tol = 2e-5 if exact else 5e-3
    for name, got, want in (("q", vw["qg"][:, :od], q), ("gate", vw["qg"][:, od:], ref["qg"][:, od:]),
                            ("k", vw["k"], k), ("v", vw["v"], v), ("act", vw["act"], ref["gated"])):
        e = normwise_err(got, want)
        say(f"    {name} normwise err {e:.2e}")
        assert e <= tol, name
    err = normwise_err(out, ref["out"])
    say(f"    block normwise err {err:.2e}")
    assert err <= (2e-5 if exact else 5e-3)
    assert np.max(np.abs(out - ref["out"])) <= (1e-4 if exact else 2e-2)


def test_long_input_odd_hidden_on_the_dense_gemm(mi355x, stream):
    """Long fp16 inputs run q, k and v as one dense MFMA GEMM launch (three weight
    segments) and o alone: a hidden size of 224 (seven 32-column stages, a partial column
    block of the o projection) and a token count that is not a multiple of the row tile;
    hidden 200 (not a whole number of stages) takes the grouped kernels instead."""
    for hidden in (224, 200):
        _long_input_case(mi355x, stream, hidden)


def _long_input_case(mi355x, stream, hidden):
    s = syn.FullAttnShape(hidden, 8, 2, 64, 0.25, 5000000.0, 1e-6)
    T = 333
    say(f"[gpu] full attention fp16, hidden {hidden}, T={T}")
    t = syn.make_full_attn_tensors(s, 79, weight_dtype=np.float16, norm_noise=0.1)
    x = syn.make_inputs(80, T, s.hidden)
    out, vw = _block(mi355x, stream, s, t, x, True)
    ref = fa.full_attn_block(x, t, spec_of(s))
    od = s.n_heads * s.head_dim
    e = normwise_err(vw["qg"][:, od:], ref["qg"][:, od:])
    say(f"    gate normwise err {e:.2e}")
    assert e <= 5e-3
    v = ref["v"].transpose(1, 0, 2).reshape(T, s.n_kv_heads * s.head_dim)
    e = normwise_err(vw["v"], v)
    say(f"    v normwise err {e:.2e}")
    assert e <= 5e-3
    err = normwise_err(out, ref["out"])
    say(f"    block normwise err {err:.2e}")
    assert err <= 5e-3 and np.max(np.abs(out - ref["out"])) <= 2e-2


@pytest.mark.parametrize("T", [1, 100, 1024, 4096])
def test_qwen3_next_size_block(mi355x, stream, T):
    s = syn.QWEN3_NEXT_FULL
    say(f"[gpu] Qwen3-Next-size full attention fp16 T={T}")
    t = syn.make_full_attn_tensors(s, 5, weight_dtype=np.float16)
    x = syn.make_inputs(6, T, s.hidden)
    out, _ = _block(mi355x, stream, s, t, x, True)
    ref = fa.full_attn_block(x, t, spec_of(s))
    err = normwise_err(out, ref["out"])
    mabs = float(np.max(np.abs(out - ref["out"])))
    say(f"    normwise err {err:.2e}; max abs {mabs:.2e}")
    assert err <= 5e-3 and mabs <= 2e-2


def test_in_place_and_argument_errors(mi355x, stream):
    s = syn.FullAttnShape(64, 4, 2, 16, 0.5, 10000.0, 1e-6)
    t = syn.make_full_attn_tensors(s, 3)
    x = syn.make_inputs(4, 21, 64)
    layer = _layer(mi355x, stream, s, t)
    lib = _lib.load()
    xb = mi355x.alloc_device(x.nbytes)
    try:
        mi355x.copy_h2d_ptr_async(xb.handle, x.ctypes.data, x.nbytes, stream)
        desc, w = layer.desc(s.eps), layer.weights()
        layer.runner.reserve(desc, 21, io=False)
        ws = layer.runner._ws
        _lib.check(lib.mx_full_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                            xb.handle, 21, ws.handle, ws.nbytes, stream))
        got = read_device(mi355x, xb.handle, np.float32, x.size, stream).reshape(x.shape)
        assert normwise_err(got, fa.full_attn_block(x, t, spec_of(s))["out"]) <= 2e-5
        assert lib.mx_full_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle, xb.handle,
                                        21, ws.handle, 16, stream) == _lib.MX_ERR_WORKSPACE
        bad = _lib.MxFullAttnDesc(64, 4, 3, 16, 4, 0, 0, 10000.0, 1e-6)  # 4 heads over 3 kv
        n = ctypes.c_size_t()
        assert lib.mx_full_attn_workspace_size(ctypes.byref(bad), 4, ctypes.byref(n)) == \
            _lib.MX_ERR_INVALID
        bad = _lib.MxFullAttnDesc(64, 4, 2, 512, 4, 0, 0, 10000.0, 1e-6)  # head_dim > 256
        assert lib.mx_full_attn_workspace_size(ctypes.byref(bad), 4, ctypes.byref(n)) == \
            _lib.MX_ERR_UNSUPPORTED
        assert lib.mx_full_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle, xb.handle,
                                        0, ws.handle, ws.nbytes, stream) == _lib.MX_OK
    finally:
        mi355x.free_device(xb)
        layer.close()


def test_in_place_fp16_long_input(mi355x, stream):
    """fp16 weights and more than 64 tokens: the residual rides in the o projection's GEMM
    epilogue (out = x + act W_o^T), which must also hold in place (out aliasing x) and give
    the out-of-place output bit for bit."""
    s = syn.FullAttnShape(256, 4, 2, 64, 0.5, 10000.0, 1e-6)
    t = syn.make_full_attn_tensors(s, 11, weight_dtype=np.float16)
    T = 100
    x = syn.make_inputs(12, T, s.hidden)
    say(f"[gpu] full attention in place, fp16 weights, T={T}")
    layer = _layer(mi355x, stream, s, t)
    lib = _lib.load()
    xb = mi355x.alloc_device(x.nbytes)
    try:
        mi355x.copy_h2d_ptr_async(xb.handle, x.ctypes.data, x.nbytes, stream)
        desc, w = layer.desc(s.eps), layer.weights()
        layer.runner.reserve(desc, T, io=False)
        ws = layer.runner._ws
        _lib.check(lib.mx_full_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                            xb.handle, T, ws.handle, ws.nbytes, stream))
        got = read_device(mi355x, xb.handle, np.float32, x.size, stream).reshape(x.shape)
        sep = layer.forward_numpy(x, s.eps)
    finally:
        mi355x.free_device(xb)
        layer.close()
    assert np.array_equal(got, sep)
    ref = fa.full_attn_block(x, t, spec_of(s))["out"]
    mabs = float(np.max(np.abs(got - ref)))
    say(f"    max abs err {mabs:.2e}")
    assert mabs <= 2e-2
