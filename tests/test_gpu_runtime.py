"""The drop-in boundary on the GPU: OffloadRuntime + MI355X backend + the MoE executors on
layers packed exactly as the reference loader packs them (contiguous, lexicographic),
chained layer after layer and compared with the oracle."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from _cases import normwise_err, spec_for
from moe_mi355x import synthetic as syn
from moe_mi355x.executors import GLM4MoeExecutor, Qwen3NextExecutor
from moe_mi355x.layout import MoeLayerLayout, make_layer_spec, pack_tensors
from moe_mi355x.runtime import OffloadRuntime
from moe_mi355x.scheduler import LookaheadScheduler
from moe_mi355x.storage import InMemoryStorage
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def build_layers(shape, n, wdt, seed):
    tensors, layers, blobs = [], [], {}
    for i in range(n):
        t = syn.make_tensors(shape, seed + i, weight_dtype=np.dtype(wdt))
        raw, meta = pack_tensors(t)  # loader packing: no padding
        layers.append(make_layer_spec(i, meta, len(raw)))
        blobs[i] = raw
        tensors.append(t)
    return tensors, layers, blobs


@pytest.mark.parametrize("arch,wdt,lookahead,pool,pinned", [
    (syn.GLM, "float32", 0, False, False),
    (syn.GLM, "float16", 2, True, True),
    (syn.QWEN, "float16", 1, True, False),
])
def test_runtime_chain_matches_oracle(mi355x, arch, wdt, lookahead, pool, pinned):
    say(f"[gpu] runtime chain {arch} {wdt} lookahead={lookahead}")
    if arch == syn.GLM:
        shape = syn.MoeShape(syn.GLM, 256, 16, 4, 128, 128, 2.5, 1e-5)
        ex = GLM4MoeExecutor(shape.config())
    else:
        shape = syn.MoeShape(syn.QWEN, 256, 32, 6, 64, 64, 1.0, 1e-6, has_bias=False,
                             has_shared_gate=True)
        ex = Qwen3NextExecutor(shape.config())
    tensors, layers, blobs = build_layers(shape, 4, wdt, 40)
    x = syn.make_inputs(40, 12, shape.hidden)
    rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(lookahead),
                        ex, use_buffer_pool=pool, use_pinned_staging=pinned)
    try:
        out, metrics = rt.run_inference([0, 1, 2, 3], x)
    finally:
        rt.close()
        ex.close()
    ref = x
    spec = spec_for(shape)
    for t in tensors:
        ref = orc.moe_block(ref, t, spec)["out"]
    err = normwise_err(out, ref)
    say(f"    normwise err {err:.2e}; overlap {metrics.overlap_ratio:.3f} "
        f"gpu_overlap {metrics.gpu_overlap_ratio:.3f}")
    assert err <= (1e-4 if wdt == "float32" else 5e-3)
    assert metrics.layer_count == 4 and metrics.transferred_bytes == sum(len(b) for b in blobs.values())
    assert all(lm.h2d_gpu_ms > 0 for lm in metrics.layer_metrics)


def test_executor_rejects_short_device_buffer(mi355x, stream):
    shape = syn.MoeShape(syn.GLM, 64, 4, 2, 32, 32, 2.5, 1e-5)
    raw, meta = pack_tensors(syn.make_tensors(shape, 1))
    layer = make_layer_spec(0, meta, len(raw))
    buf = mi355x.alloc_device(len(raw) - 16)
    ex = GLM4MoeExecutor(shape.config())
    try:
        with pytest.raises(RuntimeError, match="device buffer size"):
            ex.run_layer(layer, np.zeros((2, 64), np.float32), buf, mi355x, stream)
    finally:
        mi355x.free_device(buf)
        ex.close()


@pytest.mark.parametrize("arch,wdt,lookahead", [
    (syn.GLM, "float16", 2),
    (syn.GLM, "int8", 1),
    (syn.QWEN, "float16", 2),
])
def test_expert_granular_chain_matches_oracle(mi355x, arch, wdt, lookahead):
    """Only non-expert bytes go ahead of compute; each layer's routed experts are copied
    after its router ran.  Same outputs as the oracle, fewer bytes than whole layers."""
    from moe_mi355x.quantize import quantize_moe_tensors

    say(f"[gpu] expert-granular chain {arch} {wdt} lookahead={lookahead}")
    if arch == syn.GLM:
        shape = syn.MoeShape(syn.GLM, 256, 32, 4, 128, 128, 2.5, 1e-5)
        ex = GLM4MoeExecutor(shape.config())
    else:
        shape = syn.MoeShape(syn.QWEN, 256, 48, 6, 64, 64, 1.0, 1e-6, has_bias=False,
                             has_shared_gate=True)
        ex = Qwen3NextExecutor(shape.config())
    tensors, layers, blobs = [], [], {}
    for i in range(4):
        t = syn.make_tensors(shape, 70 + i, weight_dtype=np.float16 if wdt == "float16"
                             else np.float32)
        if wdt == "int8":
            t = quantize_moe_tensors(t)
        raw, meta = pack_tensors(t, align=16)
        layers.append(make_layer_spec(i, meta, len(raw)))
        pin = mi355x.alloc_pinned_host(len(raw))
        np.frombuffer(pin.view, dtype=np.uint8)[:] = np.frombuffer(raw, dtype=np.uint8)
        blobs[i] = pin
        tensors.append(t)
    x = syn.make_inputs(70, 3, shape.hidden)
    rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(lookahead),
                        ex, use_buffer_pool=True, expert_granular=True)
    try:
        out, metrics = rt.run_inference([0, 1, 2, 3], x)
    finally:
        rt.close()
        ex.close()
        for pin in blobs.values():
            mi355x.free_pinned_host(pin)
    ref = x
    spec = spec_for(shape)
    used, exact = 0, True
    for lay_spec, t in zip(layers, tensors):
        r = orc.moe_block(ref, t, spec)
        exact &= bool(np.all(orc.topk_margin(r["logits"], t.get("mlp.gate.e_score_correction_bias"),
                                             spec) > 1e-5))
        ref = r["out"]
        lay = MoeLayerLayout.from_meta(lay_spec.metadata["tensors"])
        ranges = lay.routed_expert_ranges()
        used += sum(b - a for a, b in lay.core_ranges(lay_spec.nbytes))
        used += sum(ranges[e][1] - ranges[e][0] for e in sorted(set(r["ids"].ravel().tolist())))
    err = normwise_err(out, ref)
    total = sum(l.nbytes for l in layers)
    say(f"    normwise err {err:.2e}; bytes {metrics.transferred_bytes} of {total}")
    assert err <= 5e-3
    assert metrics.transferred_bytes < total
    if exact:  # no near-tie routing: the copied bytes are exactly core + the oracle's experts
        assert metrics.transferred_bytes == used
    assert all(lm.h2d_gpu_ms > 0 for lm in metrics.layer_metrics)


def test_host_attention_layers_match_oracle(mi355x):
    """Full layers (attention + MoE tensors in one packed buffer): the attention runs on the
    host over only the copied-back attention tensors, the MoE step on the device."""
    from moe_mi355x.executors import host_attention

    say("[gpu] host attention + device MoE chain")
    shape = syn.MoeShape(syn.GLM, 128, 8, 2, 64, 64, 2.5, 1e-5)
    rng = np.random.default_rng(77)
    tensors, layers, blobs = [], [], {}
    for i in range(2):
        t = syn.make_tensors(shape, 70 + i, weight_dtype=np.float16)
        t["input_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        t["self_attn.o_proj.weight"] = (0.05 * rng.standard_normal((128, 128))).astype(np.float16)
        raw, meta = pack_tensors(t)
        layers.append(make_layer_spec(i, meta, len(raw)))
        blobs[i] = raw
        tensors.append(t)

    def attn(x, t):  # a stand-in attention: x + o_proj(rms_norm(x))
        h = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-5) * t["input_layernorm.weight"]
        return x + h @ t["self_attn.o_proj.weight"].astype(np.float32).T

    ex = GLM4MoeExecutor(shape.config(), attention=host_attention(attn))
    x = syn.make_inputs(71, 5, shape.hidden)
    rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(1), ex)
    try:
        out, _ = rt.run_inference([0, 1], x)
    finally:
        rt.close()
        ex.close()
    ref = x
    for t in tensors:
        ref = orc.moe_block(attn(ref, t), t, spec_for(shape))["out"]
    err = normwise_err(out, ref)
    say(f"    normwise err {err:.2e}")
    assert err <= 5e-3


@pytest.mark.parametrize("granular", [False, True])
def test_qwen_linear_attention_layers_match_oracle(mi355x, granular):
    """Full Qwen3-Next linear-attention layers (Gated DeltaNet + MoE tensors in one packed
    buffer, attn_type "linear"): both blocks on the device, chained by the runtime."""
    from oracle import linear_attn_oracle as la

    say(f"[gpu] Qwen3-Next linear-attention layers, expert_granular={granular}")
    shape = syn.MoeShape(syn.QWEN, 256, 32, 6, 64, 64, 1.0, 1e-6, has_bias=False,
                         has_shared_gate=True)
    lshape = syn.LinearAttnShape(256, 4, 32, 32, 4, 1e-6)
    tensors, layers, blobs = [], [], {}
    for i in range(3):
        t = syn.make_tensors(shape, 90 + i, weight_dtype=np.float16)
        t.update(syn.make_linear_attn_tensors(lshape, 90 + i, weight_dtype=np.float16,
                                              param_dtype=np.float32))
        raw, meta = pack_tensors(t)  # loader packing: contiguous, lexicographic
        layers.append(make_layer_spec(i, meta, len(raw), attn_type="linear"))
        pin = mi355x.alloc_pinned_host(len(raw))
        np.frombuffer(pin.view, dtype=np.uint8)[:] = np.frombuffer(raw, dtype=np.uint8)
        blobs[i] = pin
        tensors.append(t)
    cfg = shape.config()
    cfg.update(lshape.config())
    ex = Qwen3NextExecutor(cfg)
    x = syn.make_inputs(91, 9, shape.hidden)
    rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(1), ex,
                        expert_granular=granular)
    try:
        out, _ = rt.run_inference([0, 1, 2], x)
    finally:
        rt.close()
        ex.close()
        for pin in blobs.values():
            mi355x.free_pinned_host(pin)
    ref = x
    lspec = la.LinearAttnSpec(lshape.n_heads, lshape.head_dim_k, lshape.head_dim_v, lshape.eps)
    for t in tensors:
        ref = orc.moe_block(la.linear_attn_block(ref, t, lspec)["out"], t, spec_for(shape))["out"]
    err = normwise_err(out, ref)
    say(f"    normwise err {err:.2e}")
    assert err <= 5e-3


def test_qwen_hybrid_layers_match_oracle(mi355x):
    """A Qwen3-Next stack with both attention kinds (linear, linear, full) plus MoE in each
    packed layer, every block on the device, chained by the runtime."""
    from oracle import full_attn_oracle as fa
    from oracle import linear_attn_oracle as la

    say("[gpu] Qwen3-Next hybrid layers (linear, linear, full)")
    shape = syn.MoeShape(syn.QWEN, 256, 32, 6, 64, 64, 1.0, 1e-6, has_bias=False,
                         has_shared_gate=True)
    lshape = syn.LinearAttnShape(256, 4, 32, 32, 4, 1e-6)
    fshape = syn.FullAttnShape(256, 4, 2, 64, 0.25, 5000000.0, 1e-6)
    tensors, layers, blobs, kinds = [], [], {}, ["linear", "linear", "full"]
    for i, kind in enumerate(kinds):
        t = syn.make_tensors(shape, 95 + i, weight_dtype=np.float16)
        if kind == "linear":
            t.update(syn.make_linear_attn_tensors(lshape, 95 + i, weight_dtype=np.float16))
        else:
            t.update(syn.make_full_attn_tensors(fshape, 95 + i, weight_dtype=np.float16))
        raw, meta = pack_tensors(t)
        layers.append(make_layer_spec(i, meta, len(raw), attn_type=kind))
        blobs[i] = raw
        tensors.append(t)
    cfg = shape.config()
    cfg.update(lshape.config())
    cfg.update(fshape.config())
    ex = Qwen3NextExecutor(cfg)
    x = syn.make_inputs(96, 40, shape.hidden)
    rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(1), ex)
    try:
        out, _ = rt.run_inference([0, 1, 2], x)
    finally:
        rt.close()
        ex.close()
    ref = x
    lspec = la.LinearAttnSpec(lshape.n_heads, lshape.head_dim_k, lshape.head_dim_v, lshape.eps)
    fspec = fa.FullAttnSpec(fshape.n_heads, fshape.n_kv_heads, fshape.head_dim,
                            fshape.rotary_dim, fshape.rope_theta, fshape.eps)
    for kind, t in zip(kinds, tensors):
        if kind == "linear":
            ref = la.linear_attn_block(ref, t, lspec)["out"]
        else:
            ref = fa.full_attn_block(ref, t, fspec)["out"]
        ref = orc.moe_block(ref, t, spec_for(shape))["out"]
    err = normwise_err(out, ref)
    say(f"    normwise err {err:.2e}")
    assert err <= 5e-3


@pytest.mark.parametrize("arch,lookahead,resident", [
    (syn.GLM, 2, False),
    (syn.GLM, 1, True),
    (syn.QWEN, 2, True),
])
def test_device_activation_chain_equals_numpy_chain(mi355x, arch, lookahead, resident):
    """The same chain run twice: activations through NumPy after every layer (the reference
    contract) and kept on the device between layers (``device_activations=True``, no host
    wait per layer).  Outputs equal bit for bit; the first chain is checked against the
    oracle.  With ``resident`` the layers stay on the device (``DeviceResidentStorage``):
    nothing is copied and the runtime frees nothing."""
    from moe_mi355x.activations import DeviceActivations
    from moe_mi355x.storage import DeviceResidentStorage

    say(f"[gpu] device-activation chain {arch} lookahead={lookahead} resident={resident}")
    if arch == syn.GLM:
        shape = syn.MoeShape(syn.GLM, 256, 16, 4, 128, 128, 2.5, 1e-5)
        make = GLM4MoeExecutor
    else:
        shape = syn.MoeShape(syn.QWEN, 256, 32, 6, 64, 64, 1.0, 1e-6, has_bias=False,
                             has_shared_gate=True)
        make = Qwen3NextExecutor
    tensors, layers, blobs = build_layers(shape, 4, "float16", 90)
    x = syn.make_inputs(90, 20, shape.hidden)
    order = [0, 1, 2, 3, 1, 0]
    dev_bufs = {}
    st = mi355x.create_stream("resident")
    try:
        if resident:
            for i, raw in blobs.items():
                dev_bufs[i] = mi355x.alloc_device(len(raw))
                arr = np.frombuffer(raw, np.uint8)
                mi355x.copy_h2d_ptr_async(dev_bufs[i].handle, arr.ctypes.data, arr.nbytes, st)
            mi355x.synchronize_stream(st)
        outs, seen = {}, []
        for keep in (False, True):
            ex = make(shape.config(), device_activations=keep)
            storage = DeviceResidentStorage(dev_bufs) if resident else InMemoryStorage(blobs)
            rt = OffloadRuntime(layers, mi355x, storage, LookaheadScheduler(lookahead), ex,
                                use_buffer_pool=not resident)
            assert ex.stream_ordered
            orig = ex.run_layer

            def spy(layer, activations, device_weights, backend, stream, orig=orig):
                out = orig(layer, activations, device_weights, backend, stream)
                seen.append((keep, type(activations).__name__, type(out).__name__))
                return out

            ex.run_layer = spy
            try:
                out, metrics = rt.run_inference(order, x)
                ntab = len(ex._runner._tables)
            finally:
                rt.close()
                ex.close()
            assert isinstance(out, np.ndarray) and out.shape == x.shape
            assert metrics.transferred_bytes == (0 if resident else
                                                 sum(len(blobs[i]) for i in order))
            # one pointer table per (layer, device buffer): resident layers bind 4 in all
            assert ntab == 4 if resident else ntab <= 4 * (lookahead + 1)
            outs[keep] = out
        names = [s for s in seen if s[0]]
        assert names[0][1] == "ndarray" and all(s[2] == "DeviceActivations" for s in names)
        assert all(s[1] == "DeviceActivations" for s in names[1:])
        assert np.array_equal(outs[False], outs[True])
        ref = x
        spec = spec_for(shape)
        for i in order:
            ref = orc.moe_block(ref, tensors[i], spec)["out"]
        err = normwise_err(outs[False], ref)
        say(f"    normwise err vs oracle {err:.2e}; device and NumPy chains equal")
        assert err <= 5e-3
    finally:
        mi355x.synchronize_stream(st)
        for b in dev_bufs.values():
            mi355x.free_device(b)
        mi355x.destroy_stream(st)


def test_device_activations_go_stale_two_layers_later(mi355x, stream):
    """An output handle stays readable while the next layer runs and is refused once the
    layer after that has written its buffer again."""
    from moe_mi355x.activations import DeviceActivations

    shape = syn.MoeShape(syn.GLM, 128, 8, 2, 64, 64, 2.5, 1e-5)
    tensors, layers, blobs = build_layers(shape, 1, "float16", 95)
    raw = np.frombuffer(blobs[0], np.uint8)
    buf = mi355x.alloc_device(raw.nbytes)
    ex = GLM4MoeExecutor(shape.config(), device_activations=True)
    try:
        mi355x.copy_h2d_ptr_async(buf.handle, raw.ctypes.data, raw.nbytes, stream)
        x = syn.make_inputs(95, 5, shape.hidden)
        a = ex.run_layer(layers[0], x, buf, mi355x, stream)
        b = ex.run_layer(layers[0], a, buf, mi355x, stream)
        assert isinstance(a, DeviceActivations) and a.valid and b.valid
        a_host = np.asarray(a)
        ref_a = orc.moe_block(x, tensors[0], spec_for(shape))["out"]
        assert normwise_err(a_host, ref_a) <= 5e-3
        c = ex.run_layer(layers[0], b, buf, mi355x, stream)
        assert not a.valid and b.valid and c.valid
        with pytest.raises(RuntimeError, match="overwritten"):
            a.numpy()
        ref_c = orc.moe_block(orc.moe_block(ref_a, tensors[0], spec_for(shape))["out"],
                              tensors[0], spec_for(shape))["out"]
        assert normwise_err(c.numpy(), ref_c) <= 5e-3
    finally:
        ex.close()
        mi355x.free_device(buf)
