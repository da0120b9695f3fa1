"""Host side of the linear-attention block (no GPU): tensor layout parsing, ABI struct
sizes and the executor's configuration checks."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.executors import Qwen3NextExecutor
from moe_mi355x.layout import make_layer_spec, pack_tensors
from moe_mi355x.linear_attn import LinearAttnLayout, has_linear_attn


def _layer(shape, wdt=np.float16, pdt=np.float32, **kw):
    t = syn.make_linear_attn_tensors(shape, 1, weight_dtype=wdt, param_dtype=pdt)
    t.update(kw)
    raw, meta = pack_tensors(t)
    return t, meta


def test_struct_sizes_match_header():
    assert ctypes.sizeof(_lib.MxLinearAttnDesc) == 8 * 4
    assert ctypes.sizeof(_lib.MxLinearAttnWeights) == 11 * 8
    assert ctypes.sizeof(_lib.MxLinearAttnViews) == 11 * 8
    assert _lib.MX_LA_N_STAGES == len(_lib.LA_STAGE_NAMES) == 8


@pytest.mark.parametrize("shape", [syn.LinearAttnShape(8, 2, 4, 4, 4),
                                   syn.LinearAttnShape(64, 4, 16, 8, 2),
                                   syn.QWEN3_NEXT_LINEAR])
def test_layout_infers_shape(shape):
    _, meta = _layer(shape)
    lay = LinearAttnLayout.from_meta(meta)
    assert (lay.hidden, lay.n_heads, lay.head_dim_k, lay.head_dim_v, lay.conv_kernel) == (
        shape.hidden, shape.n_heads, shape.head_dim_k, shape.head_dim_v, shape.conv_kernel)
    assert lay.weight_dtype == _lib.MX_DT_F16 and lay.param_dtype == _lib.MX_DT_F32
    w = lay.weights(4096)
    by = {m["name"]: m["offset"] for m in meta}
    assert w.qkvz_w == 4096 + by["linear_attn.in_proj_qkvz.weight"]
    assert w.out_scale is None and has_linear_attn(meta)
    d = lay.desc(1e-6)
    assert (d.hidden, d.n_heads, d.head_dim_k, d.head_dim_v) == (
        shape.hidden, shape.n_heads, shape.head_dim_k, shape.head_dim_v)


def test_layout_rejects_inconsistent_tensors():
    shape = syn.LinearAttnShape(64, 4, 16, 8, 4)
    t, _ = _layer(shape)
    bad = dict(t)
    bad["linear_attn.out_proj.weight"] = np.zeros((64, 16), np.float16)
    with pytest.raises(ValueError, match="out_proj"):
        LinearAttnLayout.from_meta(pack_tensors(bad)[1])
    bad = dict(t)
    bad["linear_attn.A_log"] = bad["linear_attn.A_log"].astype(np.float16)
    with pytest.raises(ValueError, match="mixed"):
        LinearAttnLayout.from_meta(pack_tensors(bad)[1])
    bad = dict(t)
    bad["linear_attn.in_proj_qkvz.weight"] = bad["linear_attn.in_proj_qkvz.weight"].astype(np.int8)
    bad["linear_attn.in_proj_ba.weight"] = bad["linear_attn.in_proj_ba.weight"].astype(np.int8)
    bad["linear_attn.out_proj.weight"] = bad["linear_attn.out_proj.weight"].astype(np.int8)
    with pytest.raises(ValueError, match="_scale"):
        LinearAttnLayout.from_meta(pack_tensors(bad)[1])
    del t["linear_attn.dt_bias"]
    with pytest.raises(ValueError, match="lacks"):
        LinearAttnLayout.from_meta(pack_tensors(t)[1])


def test_executor_defaults_and_head_check():
    ex = Qwen3NextExecutor({"hidden_size": 64})
    # qwen3_next.py:120-125
    assert (ex.linear_num_key_heads, ex.linear_key_head_dim, ex.linear_num_value_heads,
            ex.linear_value_head_dim, ex.linear_conv_kernel_dim) == (16, 128, 32, 128, 4)
    shape = syn.LinearAttnShape(64, 4, 16, 8, 4)
    _, meta = _layer(shape)
    layer = make_layer_spec(0, meta, 0)
    with pytest.raises(ValueError, match="linear_num_key_heads == linear_num_value_heads"):
        ex.linear_attn_layout(layer)
    cfg = shape.config()
    ok = Qwen3NextExecutor(cfg)
    assert ok.linear_attn_layout(layer).n_heads == 4
    cfg["linear_value_head_dim"] = 16
    cfg["linear_key_head_dim"] = 16
    with pytest.raises(ValueError, match="config says"):
        Qwen3NextExecutor(cfg).linear_attn_layout(layer)


def test_unknown_attention_layers_need_a_hook():
    from moe_mi355x.types import DeviceBuffer

    shape = syn.MoeShape(syn.QWEN, 32, 4, 2, 16, 16, 1.0, 1e-6, has_bias=False,
                         has_shared_gate=True)
    t = syn.make_tensors(shape, 1)
    t["self_attn.c_attn.weight"] = np.zeros((8, 32), np.float32)
    raw, meta = pack_tensors(t)
    layer = make_layer_spec(0, meta, len(raw), attn_type="full")
    ex = Qwen3NextExecutor(shape.config())
    with pytest.raises(NotImplementedError, match="attention="):
        ex.run_layer(layer, np.zeros((1, 32), np.float32),
                     DeviceBuffer(handle=0, nbytes=len(raw), backend="rocm"), None, None)


def test_full_attention_layout_and_config():
    from moe_mi355x.full_attn import FullAttnLayout

    fs = syn.FullAttnShape(64, 4, 2, 16, 0.25, 10000.0, 1e-6)
    t = syn.make_full_attn_tensors(fs, 1, weight_dtype=np.float16)
    raw, meta = pack_tensors(t)
    lay = FullAttnLayout.from_meta(meta, 4, 2, 16, fs.rotary_dim, 10000.0)
    d = lay.desc(1e-6)
    assert (d.hidden, d.n_heads, d.n_kv_heads, d.head_dim, d.rotary_dim) == (64, 4, 2, 16, 4)
    assert d.weight_dtype == _lib.MX_DT_F16 and d.rope_theta == 10000.0
    assert ctypes.sizeof(_lib.MxFullAttnDesc) == 48 and ctypes.sizeof(_lib.MxFullAttnWeights) == 88
    with pytest.raises(ValueError, match="expected"):
        FullAttnLayout.from_meta(meta, 4, 4, 16, 4, 10000.0)
    del t["self_attn.v_proj.weight"]
    with pytest.raises(ValueError, match="lacks"):
        FullAttnLayout.from_meta(pack_tensors(t)[1], 4, 2, 16, 4, 10000.0)
    # executor config keys and defaults (qwen3_next.py:109-118)
    ex = Qwen3NextExecutor(fs.config())
    assert (ex.num_heads, ex.num_kv_heads, ex.head_dim, ex.rotary_dim, ex.rope_theta) == (
        4, 2, 16, 4, 10000.0)
    d = Qwen3NextExecutor({"hidden_size": 2048, "num_attention_heads": 16})
    assert (d.num_kv_heads, d.head_dim, d.rotary_dim, d.rope_theta) == (16, 128, 32, 5000000.0)
