"""The layer stream at full size: eight per-row int8 GLM-4.7 layers (3.8 GB each) in pinned
host memory, streamed through OffloadRuntime with a lookahead-2 scheduler, the device
buffer pool (three 3.8 GB buffers, each reused while copies into the others are in
flight) and the MI355X GLM4-MoE executor, both with whole-layer copies and with the
expert-granular transfer (non-expert bytes ahead, each layer's routed experts after its
router ran), at 1 and 16 tokens (runtime.py:121-198, lookahead.py:6-23).

Every layer's input and output activations are recorded at the executor boundary.  For
each layer the whole batch's routing is checked against the oracle evaluated on that
layer's recorded input (tests/_routing.py rules, from the router tensors in the host
copy), and the outputs of sampled tokens against the oracle evaluated with only their
routed experts, dequantised from the host copy of the layer.  The two transfer modes run
the same kernels on the same bytes; their outputs agree to fp32 rounding.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from _routing import check_routing_tables
from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.device_layer import DeviceMoeLayer
from moe_mi355x.executors import GLM4MoeExecutor
from moe_mi355x.layout import unpack_host
from moe_mi355x.moe import read_device
from moe_mi355x.runtime import OffloadRuntime
from moe_mi355x.scheduler import LookaheadScheduler
from moe_mi355x.storage import InMemoryStorage
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

N_LAYERS = 8  # the streaming benchmark's chain: 8 layers, 3 pooled device buffers reused
LOWP_ABS = 2e-2
SEED = 2126  # the streaming benchmark's first layer seed
PROJ = ("gate_proj", "up_proj", "down_proj")


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


class Recording:
    """Delegates to the MI355X executor and keeps, per call, a host copy of the layer's
    input and output activations and of the device's routing tables (read from the
    executor's workspace right after the synchronised call)."""

    def __init__(self, ex, backend):
        self.ex = ex
        self.backend = backend
        self.calls = []

    def _record(self, layer, activations, out):
        x = np.array(activations, np.float32)
        T, k = x.shape[0], self.ex.top_k
        E = self.ex._layout(layer).n_experts
        v = self.ex._runner.views(self.ex.moe_config(self.ex._layout(layer)).desc(), T)
        b = self.backend
        dev = {
            "ids": read_device(b, v.topk_ids, np.int32, T * k).reshape(T, k),
            "w": read_device(b, v.topk_w, np.float32, T * k).reshape(T, k),
            "counts": read_device(b, v.counts, np.int32, E),
            "offsets": read_device(b, v.offsets, np.int32, E + 1),
            "sorted_tok": read_device(b, v.sorted_tok, np.int32, T * k + T),
            "pair_pos": read_device(b, v.pair_pos, np.int32, T * k).reshape(T, k),
        }
        self.calls.append((layer.layer_id, x, np.array(out), dev))

    def run_layer(self, layer, activations, device_weights, backend, stream):
        out = self.ex.run_layer(layer, activations, device_weights, backend, stream)
        self._record(layer, activations, out)
        return out

    def run_layer_granular(self, layer, activations, device_weights, backend, stream, fetch):
        out = self.ex.run_layer_granular(layer, activations, device_weights, backend, stream,
                                         fetch)
        self._record(layer, activations, out)
        return out

    def expert_ranges(self, layer):
        return self.ex.expert_ranges(layer)

    def is_moe_layer(self, layer):
        return self.ex.is_moe_layer(layer)


@pytest.fixture(scope="module")
def int8_stream(mi355x, stream):
    G = syn.GLM47
    layers, blobs = [], {}
    say(f"[gpu] stream: building {N_LAYERS} per-row int8 GLM-4.7 layers in pinned memory")
    try:
        for i in range(N_LAYERS):
            dl = DeviceMoeLayer.synthetic(mi355x, G, SEED + i, stream, weight_dtype="int8",
                                          param_dtype="float32", layer_id=i)
            try:
                blobs[i] = dl.to_pinned()
                layers.append(dl.layer)
            finally:
                dl.close()
            say(f"    layer {i} in pinned memory ({dl.layer.nbytes / 1e9:.2f} GB)")
        yield layers, blobs
    finally:
        for pin in blobs.values():
            mi355x.free_pinned_host(pin)


@pytest.mark.parametrize("T", [1, 16])
def test_int8_layer_stream_matches_oracle(mi355x, int8_stream, T):
    G = syn.GLM47
    layers, blobs = int8_stream
    spec = orc.MoeSpec(top_k=G.top_k, router_mode=orc.SIGMOID_SELECT_BIAS, norm_topk_prob=True,
                       routed_scaling=G.routed_scaling, eps=G.eps)
    x = syn.make_inputs(SEED + 500 + T, T, G.hidden)
    outs = {}
    for mode in ("layer", "experts"):
        say(f"[gpu] stream: {N_LAYERS} int8 layers, {T} tokens, lookahead 2, {mode} transfer")
        ex = Recording(GLM4MoeExecutor(G.config(), router_mode=_lib.MX_ROUTER_SIGMOID_SELECT_BIAS,
                                       max_tokens=T), mi355x)
        rt = OffloadRuntime(layers, mi355x, InMemoryStorage(blobs), LookaheadScheduler(2), ex,
                            use_buffer_pool=True, use_pinned_staging=True,
                            expert_granular=mode == "experts")
        try:
            out, metrics = rt.run_inference(list(range(N_LAYERS)), x)
            # lookahead 2: three layer buffers in use at once, each later layer reuses one
            # whose previous layer's compute may still run when its copy is enqueued
            assert (rt._pool.misses, rt._pool.hits) == (3, N_LAYERS - 3)
        finally:
            rt.close()
            ex.ex.close()
        assert [c[0] for c in ex.calls] == list(range(N_LAYERS))
        assert np.array_equal(ex.calls[0][1], x)
        for a, b in zip(ex.calls, ex.calls[1:]):
            assert np.array_equal(a[2], b[1]), "layer input is not the previous layer's output"
        total = sum(l.nbytes for l in layers)
        if mode == "layer":
            assert metrics.transferred_bytes == total
        else:
            assert metrics.transferred_bytes < total
        say(f"    {mode}: e2e {metrics.end_to_end_seconds * 1e3:.1f} ms, copied "
            f"{metrics.transferred_bytes / 1e9:.2f} of {total / 1e9:.2f} GB")
        outs[mode] = out
        for lid, xin, xout, dev in ex.calls:
            t = unpack_host(blobs[lid].view, layers[lid].metadata["tensors"])
            h = orc.rms_norm(xin, t["post_attention_layernorm.weight"], spec.eps)
            logits = orc.router_logits(h, t)
            check_routing_tables(dev, logits, t["mlp.gate.e_score_correction_bias"], spec,
                                 G.n_experts, f"{mode} layer {lid}", has_shared=True)
            rows = np.arange(T) if T <= 4 else np.sort(
                np.random.default_rng(T + lid).choice(T, 4, replace=False))
            ref = orc.moe_block(xin[rows], t, spec, ids=dev["ids"][rows])["out"]
            err = float(np.max(np.abs(xout[rows] - ref)))
            say(f"    layer {lid}: {len(np.unique(dev['ids']))} routed experts; tokens "
                f"{rows.tolist()} max abs err {err:.3e}")
            assert err <= LOWP_ABS
    d = float(np.max(np.abs(outs["layer"] - outs["experts"])))
    say(f"    whole-layer vs expert-granular: max abs diff {d:.3e}")
    assert d <= 1e-4
