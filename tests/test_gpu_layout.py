"""MX_LAYOUT_FRAG16 on the GPU: the device converter against the host reference layout,
and the MoE block on re-tiled weights against the same block on the loader layout (the
kernels sum every product in the same order either way, so the outputs agree bit for
bit)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from _cases import spec_for
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.layout import rows_to_frag16
from moe_mi355x.moe import read_device
from moe_mi355x.quantize import quantize_moe_tensors
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

MODE_CODE = {orc.REF_SOFTMAX_BIAS: _lib.MX_ROUTER_REF_SOFTMAX_BIAS,
             orc.SIGMOID_SELECT_BIAS: _lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
             orc.SOFTMAX: _lib.MX_ROUTER_SOFTMAX}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dt,rows,cols", [(np.float16, 48, 96), (np.float16, 1536, 5120),
                                          (np.int8, 32, 256), (np.float32, 16, 48)])
def test_tile_weights_matches_host_layout(mi355x, stream, dt, rows, cols):
    say(f"[gpu] tile {np.dtype(dt).name} {rows}x{cols}")
    lib = _lib.load()
    rng = np.random.default_rng(rows + cols)
    m = (rng.standard_normal((rows, cols)) * 60).astype(dt)
    code = {np.float16: _lib.MX_DT_F16, np.int8: _lib.MX_DT_I8, np.float32: _lib.MX_DT_F32}[dt]
    src, dst = mi355x.alloc_device(m.nbytes), mi355x.alloc_device(m.nbytes)
    try:
        mi355x.copy_h2d_ptr_async(src.handle, m.ctypes.data, m.nbytes, stream)
        assert lib.mx_tile_weights(dst.handle, src.handle, rows, cols, code, stream) == 0
        got = read_device(mi355x, dst.handle, np.uint8, m.nbytes, stream)
        assert np.array_equal(got, rows_to_frag16(m))
        # rejected shapes and overlap
        assert lib.mx_tile_weights(dst.handle, src.handle, rows - 8 if rows > 16 else 8, cols,
                                   code, stream) == _lib.MX_ERR_UNSUPPORTED
        assert lib.mx_tile_weights(src.handle, src.handle, rows, cols, code,
                                   stream) == _lib.MX_ERR_INVALID
    finally:
        mi355x.free_device(src)
        mi355x.free_device(dst)


def _forward(mi355x, stream, tensors, spec, x, tiled):
    dl = DeviceMoeLayer.from_host(mi355x, tensors, stream)
    try:
        if tiled:
            dl.tile()
        cfg = dl.config(top_k=spec.top_k, router_mode=MODE_CODE[spec.router_mode],
                        routed_scaling=spec.routed_scaling, eps=spec.eps,
                        norm_topk_prob=spec.norm_topk_prob)
        out = dl.forward_numpy(cfg, x)
        if tiled:  # reads of expert weights come back in the loader layout
            n = "mlp.experts.1.down_proj.weight"
            assert np.array_equal(dl.read(n), tensors[n])
        return out
    finally:
        dl.close()


# token counts cover the decode tiles (16 rows with the K split, 32, 64) and the
# prefill tiles (128 rows, several per hot expert).
@pytest.mark.parametrize("wdt", ["float16", "int8", "float32"])
@pytest.mark.parametrize("T", [1, 5, 24, 60, 300])
def test_tiled_layer_matches_row_major(mi355x, stream, wdt, T):
    say(f"[gpu] tiled vs rows wdt={wdt} T={T}")
    shape = syn.MoeShape(syn.GLM, 256, 24, 4, 128, 64, 2.5, 1e-5)
    base = syn.make_tensors(shape, 600 + T)
    bias = np.zeros(shape.n_experts, np.float32)
    bias[:2] = [0.6, 0.3]  # a hot pair of experts: multi-tile groups at T = 300
    base["mlp.gate.e_score_correction_bias"] = bias
    if wdt == "float16":
        t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
                 else v) for n, v in base.items()}
    elif wdt == "int8":
        t = quantize_moe_tensors(base)
    else:
        t = base
    x = syn.make_inputs(600 + T, T, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    a = _forward(mi355x, stream, t, spec, x, tiled=False)
    b = _forward(mi355x, stream, t, spec, x, tiled=True)
    assert np.array_equal(a, b)


def test_tiled_layer_matches_row_major_eight_wave_blocks(mi355x, stream):
    """hidden = inter = 1024, fp16, 300 tokens: both projections run the prefill kernel's
    8-wave blocks; the narrower shared expert leaves some waves without columns."""
    say("[gpu] tiled vs rows, 8-wave prefill blocks")
    shape = syn.MoeShape(syn.GLM, 1024, 24, 4, 1024, 320, 2.5, 1e-5)
    base = syn.make_tensors(shape, 777)
    bias = np.zeros(shape.n_experts, np.float32)
    bias[:2] = [0.6, 0.3]
    base["mlp.gate.e_score_correction_bias"] = bias
    t = {n: (v.astype(np.float16) if n.startswith(("mlp.experts.", "mlp.shared_experts."))
             else v) for n, v in base.items()}
    x = syn.make_inputs(777, 300, shape.hidden)
    spec = spec_for(shape, orc.SIGMOID_SELECT_BIAS)
    a = _forward(mi355x, stream, t, spec, x, tiled=False)
    b = _forward(mi355x, stream, t, spec, x, tiled=True)
    assert np.array_equal(a, b)


def test_tile_rejects_partial_fragments(mi355x, stream):
    shape = syn.MoeShape(syn.GLM, 64, 4, 2, 40, 40, 2.5, 1e-5)  # 40 rows: no whole fragments
    t = syn.make_tensors(shape, 3, weight_dtype=np.float16)
    dl = DeviceMoeLayer.from_host(mi355x, t, stream)
    try:
        with pytest.raises(ValueError, match="fragments"):
            dl.tile()
        cfg = dl.config(top_k=2, router_mode=_lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
                        routed_scaling=2.5, eps=1e-5)
        d = cfg.desc()
        d.weight_layout = _lib.MX_LAYOUT_FRAG16  # the kernels refuse it as well
        w = dl.prepare(cfg, 4)
        dev_x = mi355x.alloc_device(4 * 64 * 4)
        try:
            # tokens = 0: the shape check comes first; nothing would be launched anyway
            rc = _lib.load().mx_expert_gate_up(ctypes.byref(d), w.experts, 0, dev_x.handle,
                                               dev_x.handle, dev_x.handle, dev_x.handle,
                                               dev_x.handle, dev_x.handle, dev_x.handle,
                                               dev_x.handle, 16, dev_x.handle, stream)
            assert rc == _lib.MX_ERR_UNSUPPORTED
        finally:
            mi355x.free_device(dev_x)
    finally:
        dl.close()
