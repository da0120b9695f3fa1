"""mx_moe_forward_noalloc (the MoE block out of the library's per-device scratch array, no
allocation) against mx_moe_forward with a caller workspace: identical outputs, bit for
bit, on two calls in a row, the second with fewer tokens (the scratch keeps the first
call's contents), for a GLM-style layer (one-token selection path included) and a
Qwen3-Next-style layer (512 experts, gated shared expert) at decode and at prefill sizes
(T >= 65: split-plane router, 128-row tiles and fp16 y rows inside the scratch)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.moe import read_device, workspace_bytes

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


CASES = {
    "glm": (syn.MoeShape(syn.GLM, 1024, 64, 8, 512, 512, 2.5, 1e-5),
            _lib.MX_ROUTER_SIGMOID_SELECT_BIAS, (64, 1)),
    "qwen": (syn.MoeShape(syn.QWEN, 1024, 512, 10, 256, 256, 1.0, 1e-6, has_bias=False,
                          has_shared_gate=True), _lib.MX_ROUTER_SOFTMAX, (48, 3)),
    # from 65 tokens: the split-plane router, 128-row m-tiles and fp16 y rows, carved out
    # of the scratch array
    "qwen_prefill": (syn.MoeShape(syn.QWEN, 1024, 512, 10, 256, 256, 1.0, 1e-6, has_bias=False,
                                  has_shared_gate=True), _lib.MX_ROUTER_SOFTMAX, (150, 70)),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_noalloc_matches_workspace_entry(mi355x, stream, name):
    shape, mode, token_counts = CASES[name]
    say(f"[gpu] no-alloc entry, {name}, tokens {token_counts}")
    lib = _lib.load()
    layer = DeviceMoeLayer.synthetic(mi355x, shape, 606, stream, weight_dtype="float16",
                                     param_dtype="float32").tile()
    cfg = layer.config(top_k=shape.top_k, router_mode=mode, routed_scaling=shape.routed_scaling,
                       eps=shape.eps)
    desc = cfg.desc()
    w = layer.prepare(cfg, max(token_counts))
    H = shape.hidden
    n = max(token_counts) * H * 4
    x_dev, out_a, out_b = (mi355x.alloc_device(n) for _ in range(3))
    try:
        for T in token_counts:
            assert workspace_bytes(desc, T) <= _lib.MX_NOALLOC_MAX_WORKSPACE
            x = syn.make_inputs(606 + T, T, H)
            mi355x.copy_h2d_ptr_async(x_dev.handle, x.ctypes.data, x.nbytes, stream)
            layer.runner.forward_device(desc, w, x_dev.handle, out_a.handle, T, stream)
            _lib.check(lib.mx_moe_forward_noalloc(ctypes.byref(desc), ctypes.byref(w),
                                                  x_dev.handle, out_b.handle, T, stream),
                       "mx_moe_forward_noalloc")
            a = read_device(mi355x, out_a.handle, np.float32, T * H, stream)
            b = read_device(mi355x, out_b.handle, np.float32, T * H, stream)
            say(f"    T={T}: max |noalloc - workspace| = {float(np.max(np.abs(a - b))):.3e}")
            assert np.all(np.isfinite(b))
            assert np.array_equal(a, b), f"T={T}: outputs differ"
    finally:
        mi355x.synchronize_stream(stream)
        for buf in (x_dev, out_a, out_b):
            mi355x.free_device(buf)
        layer.close()


def test_noalloc_rejects_batches_beyond_the_scratch(mi355x, stream):
    """A batch whose workspace exceeds the scratch is refused before anything runs."""
    G = syn.GLM47
    shape = syn.MoeShape(syn.GLM, G.hidden, G.n_experts, G.top_k, G.inter, G.shared_inter,
                         G.routed_scaling, G.eps)
    desc = _lib.MxMoeDesc(hidden=shape.hidden, inter=shape.inter,
                          shared_inter=shape.shared_inter, n_experts=shape.n_experts,
                          top_k=shape.top_k, router_mode=_lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
                          norm_topk_prob=1, weight_dtype=_lib.MX_DT_F16,
                          param_dtype=_lib.MX_DT_F32, has_bias=1, has_shared_gate=0,
                          routed_scaling=2.5, eps=1e-5, weight_layout=_lib.MX_LAYOUT_ROWS)
    T = 128
    assert workspace_bytes(desc, T) > _lib.MX_NOALLOC_MAX_WORKSPACE
    w = _lib.MxMoeWeights()
    rc = _lib.load().mx_moe_forward_noalloc(ctypes.byref(desc), ctypes.byref(w), None, None,
                                            T, stream)
    assert rc == _lib.MX_ERR_WORKSPACE
