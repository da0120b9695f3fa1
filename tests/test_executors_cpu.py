"""Executor configuration and boundary checks that need no GPU."""
from __future__ import annotations

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.backends import NullBackend
from moe_mi355x.executors import GLM4MoeExecutor, Qwen3NextExecutor
from moe_mi355x.layout import make_layer_spec, pack_tensors


def test_glm_defaults_follow_reference():
    ex = GLM4MoeExecutor({"hidden_size": 64})
    # glm4_moe.py:77-84
    assert ex.top_k == 8 and ex.n_routed_experts == 160 and ex.routed_scaling == 2.5
    assert ex.norm_topk_prob is True and ex.rms_norm_eps == 1e-5
    assert ex.router_mode == _lib.MX_ROUTER_REF_SOFTMAX_BIAS


def test_qwen_defaults_follow_reference():
    ex = Qwen3NextExecutor({"hidden_size": 64})
    # qwen3_next.py:108, :127-133
    assert ex.top_k == 10 and ex.num_experts == 512 and ex.rms_norm_eps == 1e-6
    assert ex.routed_scaling == 1.0 and ex.router_mode == _lib.MX_ROUTER_SOFTMAX


def test_moe_config_from_layer():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    _, meta = pack_tensors(syn.make_tensors(shape, 1), align=16)
    layer = make_layer_spec(3, meta, 0)
    ex = GLM4MoeExecutor(shape.config(), router_mode="sigmoid_select_bias")
    cfg = ex.moe_config(ex._layout(layer))
    d = cfg.desc()
    assert (d.hidden, d.inter, d.shared_inter, d.n_experts, d.top_k) == (32, 16, 16, 4, 2)
    assert d.router_mode == _lib.MX_ROUTER_SIGMOID_SELECT_BIAS and d.has_bias == 1
    assert d.routed_scaling == pytest.approx(2.5)


def test_run_layer_requires_the_rocm_backend():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    raw, meta = pack_tensors(syn.make_tensors(shape, 1), align=16)
    layer = make_layer_spec(0, meta, len(raw))
    be = NullBackend()
    buf = be.alloc_device(len(raw))
    ex = GLM4MoeExecutor(shape.config())
    with pytest.raises(RuntimeError, match="MI355X backend"):
        ex.run_layer(layer, np.zeros((2, 32), np.float32), buf, be, be.create_stream("c"))


def test_attention_layers_need_an_attention_callable():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 1)
    t["self_attn.q_proj.weight"] = np.zeros((32, 32), np.float32)
    raw, meta = pack_tensors(t, align=16)
    layer = make_layer_spec(0, meta, len(raw))
    be = NullBackend()
    ex = GLM4MoeExecutor(shape.config())
    with pytest.raises(NotImplementedError, match="attention"):
        ex.run_layer(layer, np.zeros((2, 32), np.float32), be.alloc_device(len(raw)), be, None)
    seen = []

    def attention(x, layer_, dw, backend, stream):
        seen.append(layer_.layer_id)
        raise KeyError("stop")  # reached the hook; the MoE step is not run on CPU

    ex2 = GLM4MoeExecutor(shape.config(), attention=attention)
    with pytest.raises(KeyError):
        ex2.run_layer(layer, np.zeros((2, 32), np.float32), be.alloc_device(len(raw)), be, None)
    assert seen == [0]


def test_embed_and_lm_head():
    ex = GLM4MoeExecutor({"hidden_size": 4})
    emb = np.arange(12, dtype=np.float16).reshape(3, 4)
    out = ex.embed([2, 0], emb)
    assert out.dtype == np.float32 and out.tolist() == [[8, 9, 10, 11], [0, 1, 2, 3]]
    h = np.ones((1, 4), np.float32)
    logits = ex.lm_head(h, np.ones(4, np.float32), np.eye(4, dtype=np.float32))
    np.testing.assert_allclose(logits, np.ones((1, 4)), rtol=1e-5)
