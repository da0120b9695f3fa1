"""The linear-attention (Gated DeltaNet) block on the GPU against the oracle
(oracle/linear_attn_oracle.py, itself pinned to the reference's golden outputs)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from _cases import GOLDEN, normwise_err
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.linear_attn import DeviceLinearAttnLayer
from moe_mi355x.moe import read_device
from moe_mi355x.quantize import quantize_rows_int8
from oracle import linear_attn_oracle as la

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def spec_of(shape):
    return la.LinearAttnSpec(shape.n_heads, shape.head_dim_k, shape.head_dim_v, shape.eps)


def upload(mi355x, stream, arr):
    arr = np.ascontiguousarray(arr)
    buf = mi355x.alloc_device(max(arr.nbytes, 16))
    mi355x.copy_h2d_ptr_async(buf.handle, arr.ctypes.data, arr.nbytes, stream)
    mi355x.synchronize_stream(stream)
    return buf


@pytest.mark.parametrize("n,dk,dv,T,gs", [
    (2, 4, 4, 3, 0.2), (3, 8, 12, 17, 0.2), (4, 16, 8, 33, 0.2), (2, 32, 40, 50, 0.2),
    (2, 64, 64, 1, 0.2), (4, 128, 128, 37, 0.2), (2, 128, 96, 16, 0.2), (1, 256, 64, 21, 0.2),
    (1, 512, 32, 9, 0.2),
    # from 64 tokens the chunked form on MFMA: whole and partial chunks, the four head
    # shapes it is built for, a shape it is not (sequential), strong and mixed decays
    (2, 128, 128, 64, 0.2), (3, 128, 128, 200, 0.2), (2, 64, 64, 130, 0.2),
    (1, 128, 64, 150, 0.2), (2, 64, 128, 300, 0.2), (2, 128, 96, 100, 0.2),
    (2, 128, 128, 257, 3.0), (1, 64, 64, 1000, 0.05),
])
def test_scan_matches_oracle(mi355x, stream, n, dk, dv, T, gs):
    say(f"[gpu] scan n={n} dk={dk} dv={dv} T={T} decay scale {gs}")
    rng = np.random.default_rng(n * 1000 + dk + T)
    q = rng.standard_normal((T, n * dk)).astype(np.float32)
    kb = (rng.standard_normal((T, n * dk)) * 0.3).astype(np.float32)
    v = rng.standard_normal((T, n * dv)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((T, n))) * gs).astype(np.float32)
    decay = np.exp(g).astype(np.float32)
    ref = la.gated_recurrence(q, kb, v, g, n, dk, dv)
    for form in ("sequential", "workspace"):
        got = run_scan(mi355x, stream, (q, kb, v, decay), T, n, dk, dv, form)
        err = normwise_err(got, ref)
        say(f"    {form}: normwise err {err:.2e}")
        assert err <= 1e-5


def run_scan(mi355x, stream, arrays, T, n, dk, dv, form):
    """mx_gated_delta_scan (token-sequential) or mx_gated_delta_scan_ws (chunked from 64
    tokens for heads of 64 / 128) on uploaded copies of ``arrays``."""
    lib = _lib.load()
    bufs = [upload(mi355x, stream, a) for a in arrays]
    o = mi355x.alloc_device(T * n * dv * 4)
    ws = None
    try:
        if form == "sequential":
            _lib.check(lib.mx_gated_delta_scan(*(b.handle for b in bufs), T, n, dk, dv,
                                               o.handle, stream))
        else:
            nb = ctypes.c_size_t()
            _lib.check(lib.mx_gated_delta_scan_workspace_size(T, n, dk, dv, ctypes.byref(nb)))
            chunked = T >= 64 and dk in (64, 128) and dv in (64, 128)
            assert (nb.value > 0) == chunked
            ws = mi355x.alloc_device(max(nb.value, 16))
            if nb.value:
                rc = lib.mx_gated_delta_scan_ws(*(b.handle for b in bufs), T, n, dk, dv,
                                                o.handle, ws.handle, nb.value - 4, stream)
                assert rc == _lib.MX_ERR_WORKSPACE
            _lib.check(lib.mx_gated_delta_scan_ws(*(b.handle for b in bufs), T, n, dk, dv,
                                                  o.handle, ws.handle, nb.value, stream))
        return read_device(mi355x, o.handle, np.float32, T * n * dv, stream).reshape(T, -1)
    finally:
        for b in bufs + [o] + ([ws] if ws is not None else []):
            mi355x.free_device(b)


@pytest.mark.parametrize("T", [70, 300])
def test_chunked_scan_zero_and_tiny_decays(mi355x, stream, T):
    """Decays that underflow to zero (the state restarts there, inside a chunk and on a
    chunk's first token) and tiny nonzero ones between ordinary ones."""
    n, dk, dv = 2, 128, 128
    say(f"[gpu] chunked scan with zero decays, T={T}")
    rng = np.random.default_rng(77 + T)
    q = rng.standard_normal((T, n * dk)).astype(np.float32)
    kb = (rng.standard_normal((T, n * dk)) * 0.3).astype(np.float32)
    v = rng.standard_normal((T, n * dv)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((T, n))) * 0.3).astype(np.float32)
    g[5, 0] = g[64 % T, 1] = g[T - 2, 0] = -200.0      # exp -> 0 in fp32
    g[10, 1] = g[40, 0] = -80.0                         # exp -> ~1.8e-35
    g[11:20, 1] = -0.01
    decay = np.exp(g).astype(np.float32)
    assert decay[5, 0] == 0.0 and decay[10, 1] > 0.0
    with np.errstate(divide="ignore"):
        ref = la.gated_recurrence(q, kb, v, np.log(decay), n, dk, dv)
    got = run_scan(mi355x, stream, (q, kb, v, decay), T, n, dk, dv, "workspace")
    err = normwise_err(got, ref)
    say(f"    normwise err {err:.2e}")
    assert np.all(np.isfinite(got)) and err <= 1e-5


def _block(mi355x, stream, shape, t, x):
    layer = DeviceLinearAttnLayer.from_host(mi355x, t, stream)
    try:
        out = layer.forward_numpy(x, shape.eps)
        T = x.shape[0]
        v = layer.runner.views(layer.desc(shape.eps), T)
        n, dk, dv = shape.n_heads, shape.head_dim_k, shape.head_dim_v
        views = {
            "qkvz": read_device(mi355x, v.qkvz, np.float32, T * shape.qkvz_rows, stream),
            "ba": read_device(mi355x, v.ba, np.float32, T * shape.ba_rows, stream),
            "q": read_device(mi355x, v.q, np.float32, T * n * dk, stream),
            "kb": read_device(mi355x, v.kb, np.float32, T * n * dk, stream),
            "v": read_device(mi355x, v.v, np.float32, T * n * dv, stream),
            "decay": read_device(mi355x, v.decay, np.float32, T * n, stream),
            "o": read_device(mi355x, v.o, np.float32, T * n * dv, stream),
        }
        return out, {k: a.reshape(T, -1) for k, a in views.items()}
    finally:
        layer.close()


def _golden_cases():
    import json
    p = GOLDEN / "linear_attn_index.json"
    return json.loads(p.read_text()) if p.exists() else {}


@pytest.mark.parametrize("name", sorted(_golden_cases()))
def test_block_matches_reference_golden(mi355x, stream, name):
    case = _golden_cases()[name]
    shape = syn.LinearAttnShape(**case["shape"])
    say(f"[gpu] linear attention golden {name} {shape}")
    dt = np.dtype(case["dtype"])
    t = syn.make_linear_attn_tensors(shape, case["seed"], weight_dtype=dt, param_dtype=dt,
                                     norm_noise=case["norm_noise"])
    x = syn.make_inputs(case["seed"], case["tokens"], shape.hidden)
    if shape.hidden % 8 and dt == np.float16:
        pytest.skip("fp16 projections need hidden % 8 == 0")
    out, _ = _block(mi355x, stream, shape, t, x)
    want = np.load(GOLDEN / f"{name}.npz")["out"]
    err = float(np.max(np.abs(out - want)))
    say(f"    max abs err vs reference {err:.2e}")
    assert err <= (1e-4 if dt == np.float32 else 2e-2)


@pytest.mark.parametrize("wdt,T", [("float32", 5), ("float32", 130), ("float16", 1),
                                   ("float16", 24), ("float16", 300), ("int8", 7),
                                   ("int8", 200)])
def test_block_intermediates_match_oracle(mi355x, stream, wdt, T):
    shape = syn.LinearAttnShape(256, 4, 64, 32, 4, 1e-6)
    say(f"[gpu] linear attention {wdt} T={T}")
    t = syn.make_linear_attn_tensors(shape, 50 + T, weight_dtype=np.float16 if wdt == "int8"
                                     else np.dtype(wdt), param_dtype=np.float32, norm_noise=0.1)
    ref_t = dict(t)
    if wdt == "int8":
        for k in (la.QKVZ, la.BA, la.OUT):
            qv, s = quantize_rows_int8(t[k].astype(np.float32))
            t[k], t[k + "_scale"] = qv, s
            ref_t[k] = qv.astype(np.float32) * s.astype(np.float32)[:, None]
    x = syn.make_inputs(60 + T, T, shape.hidden)
    out, views = _block(mi355x, stream, shape, t, x)
    ref = la.linear_attn_block(x, ref_t, spec_of(shape))
    exact = wdt == "float32"
    tol = {"qkvz": 1e-5 if exact else 3e-3, "ba": 1e-5 if exact else 3e-3}
    for k in ("qkvz", "ba"):
        e = normwise_err(views[k], ref[k])
        say(f"    {k} normwise err {e:.2e}")
        assert e <= tol[k], k
    # the conv/gate/scan stages from the device's own projections: fp32 work throughout
    qkvz, ba = views["qkvz"], views["ba"]
    n, dk, dv = shape.n_heads, shape.head_dim_k, shape.head_dim_v
    qd, vd = n * dk, n * dv
    conv = la.silu(la.causal_conv1d(qkvz[:, : 2 * qd + vd], t[la.CONV].squeeze(1)))
    kb = la.sigmoid(ba[:, :qd]) * conv[:, qd: 2 * qd]
    g = -np.exp(t[la.A_LOG]) * la.softplus(ba[:, qd:] + t[la.DT_BIAS])
    for k, want in (("q", conv[:, :qd]), ("kb", kb), ("v", conv[:, 2 * qd:]),
                    ("decay", np.exp(g))):
        e = normwise_err(views[k], want)
        assert e <= 2e-6, (k, e)
    o = la.gated_recurrence(views["q"], views["kb"], views["v"], np.log(views["decay"]),
                            n, dk, dv)
    e = normwise_err(views["o"], o)
    say(f"    scan normwise err {e:.2e}")
    assert e <= 1e-5
    err = normwise_err(out, ref["out"])
    say(f"    block normwise err {err:.2e}; max abs {np.max(np.abs(out - ref['out'])):.2e}")
    assert err <= (2e-5 if exact else 5e-3)
    assert np.max(np.abs(out - ref["out"])) <= (1e-4 if exact else 2e-2)


def test_long_input_odd_hidden_on_the_dense_gemm(mi355x, stream):
    """Long fp16 inputs run the projections on the dense MFMA GEMM (qkvz and ba in one
    launch): a hidden size of 224 (seven 32-column stages, and a partial column block of the
    out projection), a token count that is not a multiple of the 128 / 256-row tile, and the
    ba segment's partial column block; hidden 200 (not a whole number of 32-column stages)
    takes the grouped kernels instead."""
    for hidden in (224, 200):
        _long_input_case(mi355x, stream, hidden)


def _long_input_case(mi355x, stream, hidden):
    shape = syn.LinearAttnShape(hidden, 4, 64, 32, 4, 1e-6)
    T = 333
    say(f"[gpu] linear attention fp16, hidden {hidden}, T={T}")
    t = syn.make_linear_attn_tensors(shape, 77, weight_dtype=np.float16, param_dtype=np.float32,
                                     norm_noise=0.1)
    x = syn.make_inputs(78, T, shape.hidden)
    out, views = _block(mi355x, stream, shape, t, x)
    ref = la.linear_attn_block(x, t, spec_of(shape))
    for k in ("qkvz", "ba"):
        e = normwise_err(views[k], ref[k])
        say(f"    {k} normwise err {e:.2e}")
        assert e <= 3e-3, k
    err = normwise_err(out, ref["out"])
    assert err <= 5e-3 and np.max(np.abs(out - ref["out"])) <= 2e-2


@pytest.mark.parametrize("T", [1, 64, 512, 4096])
def test_qwen3_next_size_block(mi355x, stream, T):
    shape = syn.QWEN3_NEXT_LINEAR
    say(f"[gpu] Qwen3-Next-size linear attention fp16 T={T}")
    t = syn.make_linear_attn_tensors(shape, 7, weight_dtype=np.float16, param_dtype=np.float32)
    x = syn.make_inputs(8, T, shape.hidden)
    out, views = _block(mi355x, stream, shape, t, x)
    ref = la.linear_attn_block(x, t, spec_of(shape))
    err = normwise_err(out, ref["out"])
    mabs = float(np.max(np.abs(out - ref["out"])))
    say(f"    normwise err {err:.2e}; max abs {mabs:.2e}")
    assert err <= 5e-3 and mabs <= 2e-2


def test_in_place_and_argument_errors(mi355x, stream):
    shape = syn.LinearAttnShape(64, 2, 16, 16, 4, 1e-6)
    t = syn.make_linear_attn_tensors(shape, 3)
    x = syn.make_inputs(4, 6, shape.hidden)
    layer = DeviceLinearAttnLayer.from_host(mi355x, t, stream)
    lib = _lib.load()
    xb = upload(mi355x, stream, x)
    try:
        desc, w = layer.desc(shape.eps), layer.weights()
        layer.runner.reserve(desc, 6, io=False)
        ws = layer.runner._ws
        _lib.check(lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                              xb.handle, 6, ws.handle, ws.nbytes, stream))
        got = read_device(mi355x, xb.handle, np.float32, x.size, stream).reshape(x.shape)
        ref = la.linear_attn_block(x, t, spec_of(shape))["out"]
        assert normwise_err(got, ref) <= 2e-5
        assert lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                          xb.handle, 6, ws.handle, 16, stream) == \
            _lib.MX_ERR_WORKSPACE
        bad = _lib.MxLinearAttnDesc(64, 2, 12, 16, 4, 0, 0, 1e-6)  # dk not a power of two
        n = ctypes.c_size_t()
        assert lib.mx_linear_attn_workspace_size(ctypes.byref(bad), 6, ctypes.byref(n)) == \
            _lib.MX_ERR_UNSUPPORTED
        nw = _lib.MxLinearAttnWeights()
        assert lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(nw), xb.handle,
                                          xb.handle, 6, ws.handle, ws.nbytes, stream) == \
            _lib.MX_ERR_INVALID
        assert lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                          xb.handle, 0, ws.handle, ws.nbytes, stream) == _lib.MX_OK
    finally:
        mi355x.free_device(xb)
        layer.close()


def test_in_place_fp16_long_input(mi355x, stream):
    """fp16 weights and more than 64 tokens: the residual rides in the out projection's GEMM
    epilogue (out = x + act W_out^T), which must also hold in place (out aliasing x) and give
    the out-of-place output bit for bit."""
    shape = syn.LinearAttnShape(256, 4, 32, 32, 4, 1e-6)
    t = syn.make_linear_attn_tensors(shape, 13, weight_dtype=np.float16)
    T = 100
    x = syn.make_inputs(14, T, shape.hidden)
    say(f"[gpu] linear attention in place, fp16 weights, T={T}")
    layer = DeviceLinearAttnLayer.from_host(mi355x, t, stream)
    lib = _lib.load()
    xb = upload(mi355x, stream, x)
    try:
        desc, w = layer.desc(shape.eps), layer.weights()
        layer.runner.reserve(desc, T, io=False)
        ws = layer.runner._ws
        _lib.check(lib.mx_linear_attn_forward(ctypes.byref(desc), ctypes.byref(w), xb.handle,
                                              xb.handle, T, ws.handle, ws.nbytes, stream))
        got = read_device(mi355x, xb.handle, np.float32, x.size, stream).reshape(x.shape)
        sep = layer.forward_numpy(x, shape.eps)
    finally:
        mi355x.free_device(xb)
        layer.close()
    assert np.array_equal(got, sep)
    ref = la.linear_attn_block(x, t, spec_of(shape))["out"]
    mabs = float(np.max(np.abs(got - ref)))
    say(f"    max abs err {mabs:.2e}")
    assert mabs <= 2e-2
