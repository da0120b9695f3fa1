"""Executor configuration and boundary checks that need no GPU."""
from __future__ import annotations

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from host_backend import HostArenaBackend
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
    be = HostArenaBackend()
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
    be = HostArenaBackend()
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


def _attention_layer(seed=5):
    rng = np.random.default_rng(seed)
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 1)
    t["input_layernorm.weight"] = rng.standard_normal(32).astype(np.float32)
    t["self_attn.q_proj.weight"] = rng.standard_normal((32, 32)).astype(np.float16)
    t["self_attn.o_proj.weight"] = rng.standard_normal((32, 32)).astype(np.float32)
    buf, meta = pack_tensors(t, align=16)
    return t, buf, make_layer_spec(0, meta, len(buf))


class _PtrBackend(HostArenaBackend):
    """HostArenaBackend with pointer D2H copies over one numpy array; logs the byte counts."""

    def __init__(self, data):
        super().__init__()
        self.data = np.frombuffer(bytes(data), np.uint8)
        self.copied = []

    def copy_d2h_ptr_async(self, dst_addr, src, nbytes, stream):
        import ctypes
        ctypes.memmove(dst_addr, self.data.ctypes.data + src, nbytes)
        self.copied.append(nbytes)


def test_read_layer_tensors_copies_only_non_mlp_ranges():
    from moe_mi355x.executors import DeviceBuffer, read_layer_tensors

    t, buf, layer = _attention_layer()
    be = _PtrBackend(buf)
    dev = DeviceBuffer(handle=0, nbytes=len(buf), backend="null")
    got = read_layer_tensors(layer, dev, be, None, gap=1)
    assert set(got) == {"input_layernorm.weight", "self_attn.q_proj.weight",
                        "self_attn.o_proj.weight"}
    for n, v in got.items():
        assert v.dtype == t[n].dtype and np.array_equal(v, t[n])
    want = sum(t[n].nbytes for n in got)
    assert want <= sum(be.copied) < len(buf) // 4
    # the whole-layer fallback of backends without pointer copies gives the same tensors
    nb = HostArenaBackend()
    d2 = nb.alloc_device(len(buf))
    from moe_mi355x.types import HostBuffer
    nb.copy_h2d_async(d2, HostBuffer(view=memoryview(buf)), None)
    got2 = read_layer_tensors(layer, d2, nb, None)
    assert all(np.array_equal(got2[n], got[n]) for n in got)


def test_merge_ranges():
    from moe_mi355x.executors import _merge_ranges

    assert _merge_ranges([(10, 20), (0, 5), (21, 30), (100, 110)], gap=2) == [
        (0, 5), (10, 30), (100, 110)]
    assert _merge_ranges([(0, 5), (3, 4)], gap=0) == [(0, 5)]


def test_host_attention_hook_runs_before_the_moe_step():
    from moe_mi355x.executors import DeviceBuffer, host_attention

    t, buf, layer = _attention_layer()
    seen = {}

    def attn(x, tensors):
        seen.update(tensors)
        return x + tensors["input_layernorm.weight"]

    hook = host_attention(attn)
    be = _PtrBackend(buf)
    x = np.zeros((3, 32), np.float32)
    y = hook(x, layer, DeviceBuffer(handle=0, nbytes=len(buf), backend="null"), be, None)
    assert np.array_equal(y, np.broadcast_to(t["input_layernorm.weight"], (3, 32)))
    assert "self_attn.o_proj.weight" in seen and not any(n.startswith("mlp.") for n in seen)


def _dense_layer(is_moe=None, seed=7):
    """A GLM4 dense (first_k_dense_replace) layer: attention tensors + a dense SwiGLU MLP."""
    rng = np.random.default_rng(seed)
    H, inter = 32, 48
    t = {
        "input_layernorm.weight": rng.standard_normal(H).astype(np.float32),
        "self_attn.o_proj.weight": rng.standard_normal((H, H)).astype(np.float32),
        "post_attention_layernorm.weight": rng.standard_normal(H).astype(np.float32),
        "mlp.gate_proj.weight": (0.1 * rng.standard_normal((inter, H))).astype(np.float32),
        "mlp.up_proj.weight": (0.1 * rng.standard_normal((inter, H))).astype(np.float32),
        "mlp.down_proj.weight": (0.1 * rng.standard_normal((H, inter))).astype(np.float32),
    }
    buf, meta = pack_tensors(t)
    layer = make_layer_spec(0, meta, len(buf))
    del layer.metadata["is_moe"]
    if is_moe is not None:
        layer.metadata["is_moe"] = is_moe
    return t, buf, layer


def _dense_mlp(x, t, eps=1e-5):
    # glm4_moe.py:166-172 restated: x + down(silu(gate(h)) * up(h)), h = rms_norm(x)
    h = t["post_attention_layernorm.weight"] * (x / np.sqrt(np.mean(x * x, -1, keepdims=True) + eps))
    g = h @ t["mlp.gate_proj.weight"].T
    u = h @ t["mlp.up_proj.weight"].T
    return x + ((g / (1 + np.exp(-g))) * u) @ t["mlp.down_proj.weight"].T


@pytest.mark.parametrize("is_moe", [None, False])
def test_glm_layer_without_is_moe_is_a_dense_layer(is_moe):
    """glm4_moe.py:102 defaults is_moe to False: such layers take the dense hook."""
    from moe_mi355x.executors import DeviceBuffer, host_attention, host_dense

    t, buf, layer = _dense_layer(is_moe)
    cfg = {"hidden_size": 32}
    be = _PtrBackend(buf)
    dev = DeviceBuffer(handle=0, nbytes=len(buf), backend="null")
    x = np.random.default_rng(1).standard_normal((3, 32)).astype(np.float32)
    attn = host_attention(lambda x_, tt: x_ + tt["input_layernorm.weight"])
    ex = GLM4MoeExecutor(cfg, attention=attn)
    assert not ex.is_moe_layer(layer)
    with pytest.raises(NotImplementedError, match="dense"):
        ex.run_layer(layer, x, dev, be, None)
    seen = {}

    def dense(x_, tt):
        seen.update(tt)
        return _dense_mlp(x_, tt)

    ex2 = GLM4MoeExecutor(cfg, attention=attn, dense=host_dense(dense))
    y = ex2.run_layer(layer, x, dev, be, None)
    assert set(seen) == {"post_attention_layernorm.weight", "mlp.gate_proj.weight",
                         "mlp.up_proj.weight", "mlp.down_proj.weight"}
    want = _dense_mlp(x + t["input_layernorm.weight"], t)
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6)


def test_moe_flag_per_executor():
    _, _, layer = _dense_layer(None)
    assert not GLM4MoeExecutor({"hidden_size": 32}).is_moe_layer(layer)
    layer.metadata["is_moe"] = True
    assert GLM4MoeExecutor({"hidden_size": 32}).is_moe_layer(layer)
    # Qwen3-Next runs its MoE block on every layer (qwen3_next.py:155-156).
    del layer.metadata["is_moe"]
    assert Qwen3NextExecutor({"hidden_size": 32}).is_moe_layer(layer)


def test_detect_backend_has_no_cpu_fallback():
    from moe_mi355x.backends import detect_backend

    with pytest.raises(RuntimeError):
        detect_backend(10 ** 6)
