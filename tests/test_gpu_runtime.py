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
from moe_mi355x.layout import make_layer_spec, pack_tensors
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
