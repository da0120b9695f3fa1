"""Packed layer layout (loader contract, loader/huggingface.py:458-591 of the reference),
metadata parsing and the device pointer table."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest

from moe_mi355x import _lib
from moe_mi355x import synthetic as syn
from moe_mi355x.layout import MoeLayerLayout, pack_tensors, unpack_host
from moe_mi355x.quantize import quantize_moe_tensors


def test_pack_is_lexicographic_and_contiguous():
    t = {"b": np.arange(3, dtype=np.float32), "a": np.ones((2, 2), np.float16),
         "mlp.experts.10.x": np.zeros(1, np.int8), "mlp.experts.2.x": np.zeros(1, np.int8)}
    raw, meta = pack_tensors(t)
    assert [m["name"] for m in meta] == ["a", "b", "mlp.experts.10.x", "mlp.experts.2.x"]
    assert [m["offset"] for m in meta] == [0, 8, 20, 21]
    back = unpack_host(raw, meta)
    for k, v in t.items():
        assert np.array_equal(back[k], v) and back[k].dtype == v.dtype


def test_pack_alignment():
    t = {"a": np.zeros(3, np.int8), "b": np.zeros(5, np.float32)}
    _, meta = pack_tensors(t, align=256)
    assert meta[1]["offset"] == 256


@pytest.mark.parametrize("shape", [syn.C1, syn.MoeShape(syn.QWEN, 64, 6, 2, 32, 16, 1.0, 1e-6,
                                                        has_bias=False, has_shared_gate=True)])
def test_layout_parses_both_architectures(shape):
    t = syn.make_tensors(shape, 1) if shape.hidden < 1024 else \
        {n: np.zeros(s, np.float32) for n, s, _, _ in syn.tensor_specs(shape)}
    _, meta = pack_tensors(t, align=16)
    lay = MoeLayerLayout.from_meta(meta)
    assert (lay.hidden, lay.inter, lay.shared_inter, lay.n_experts) == \
        (shape.hidden, shape.inter, shape.shared_inter, shape.n_experts)
    assert lay.has_bias == shape.has_bias and lay.has_shared_gate == shape.has_shared_gate
    assert lay.weight_dtype == _lib.MX_DT_F32 and lay.param_dtype == _lib.MX_DT_F32
    base = 1 << 40
    table = lay.expert_table(base)
    assert len(table) == shape.n_experts + 1
    e1 = [m for m in meta if m["name"] == "mlp.experts.1.down_proj.weight"][0]
    assert table[1].down == base + e1["offset"]
    assert table[shape.n_experts].gate is not None  # shared expert in the last slot
    w = lay.weights(base, 1234)
    assert w.experts == 1234 and w.norm_w == base + lay.offset("post_attention_layernorm.weight")
    assert (w.bias is not None) == shape.has_bias


def test_int8_layout_carries_scales():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = quantize_moe_tensors(syn.make_tensors(shape, 2))
    _, meta = pack_tensors(t, align=16)
    lay = MoeLayerLayout.from_meta(meta)
    assert lay.weight_dtype == _lib.MX_DT_I8
    table = lay.expert_table(4096)
    assert table[0].gate_scale == 4096 + lay.offset("mlp.experts.0.gate_proj.weight_scale")


def test_layout_errors():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 3)
    bad = dict(t)
    del bad["mlp.experts.2.up_proj.weight"]
    with pytest.raises(ValueError, match="expert 2"):
        MoeLayerLayout.from_meta(pack_tensors(bad)[1])
    bad = dict(t)
    bad["mlp.experts.1.gate_proj.weight"] = bad["mlp.experts.1.gate_proj.weight"].astype(np.float16)
    with pytest.raises(ValueError, match="one dtype"):
        MoeLayerLayout.from_meta(pack_tensors(bad)[1])
    bad = dict(t)
    del bad["mlp.gate.weight"]
    with pytest.raises(ValueError, match="missing"):
        MoeLayerLayout.from_meta(pack_tensors(bad)[1])
    q = quantize_moe_tensors(t)
    del q["mlp.experts.0.down_proj.weight_scale"]
    with pytest.raises(ValueError, match="scale"):
        MoeLayerLayout.from_meta(pack_tensors(q)[1])


def test_misaligned_expert_is_reported():
    shape = syn.MoeShape(syn.GLM, 32, 4, 2, 16, 16, 2.5, 1e-5)
    t = syn.make_tensors(shape, 4)
    t["mlp.a_odd"] = np.zeros(3, np.int8)  # sorts before the experts and shifts them by 3 bytes
    _, meta = pack_tensors(t)
    lay = MoeLayerLayout.from_meta(meta)
    with pytest.raises(ValueError, match="16-byte aligned"):
        lay.expert_table(0)


def test_expert_ptrs_struct_matches_header():
    assert ctypes.sizeof(_lib.MxExpertPtrs) == 48
    assert ctypes.sizeof(_lib.MxMoeDesc) == 14 * 4


# ---- MX_LAYOUT_FRAG16 host reference (the device converter is checked against it) -------

@pytest.mark.parametrize("dt,cols", [(np.float16, 64), (np.float16, 96), (np.int8, 128),
                                     (np.float32, 48)])
def test_frag16_round_trip_and_placement(dt, cols):
    from moe_mi355x.layout import frag16_to_rows, rows_to_frag16
    rng = np.random.default_rng(cols)
    m = (rng.standard_normal((48, cols)) * 50).astype(dt)
    t = rows_to_frag16(m)
    assert t.nbytes == m.nbytes
    assert np.array_equal(frag16_to_rows(t, 48, cols, dt).view(np.uint8), m.view(np.uint8))
    rb = m.view(np.uint8).reshape(48, -1)
    nch = rb.shape[1] // 64
    frags = t.reshape(-1, 64, 16)
    # every 16-byte piece: fragment (g, c), lane 16 q + j <- row 16 g + j, bytes 64 c + 16 q
    for g in range(3):
        for c in range(nch):
            for q in range(4):
                for j in range(16):
                    assert np.array_equal(frags[g * nch + c, 16 * q + j],
                                          rb[16 * g + j, 64 * c + 16 * q: 64 * c + 16 * q + 16])


def test_frag16_rejects_partial_fragments():
    from moe_mi355x.layout import rows_to_frag16
    with pytest.raises(ValueError):
        rows_to_frag16(np.zeros((24, 64), np.float16))
    with pytest.raises(ValueError):
        rows_to_frag16(np.zeros((16, 40), np.float16))


def test_layout_constants_match_header():
    hdr = (Path(__file__).resolve().parents[1] / "include" / "moe_mi355x.h").read_text()
    assert "#define MX_LAYOUT_ROWS 0" in hdr and "#define MX_LAYOUT_FRAG16 1" in hdr
    assert _lib.MX_LAYOUT_ROWS == 0 and _lib.MX_LAYOUT_FRAG16 == 1


# ---- byte ranges for expert-granular transfer ---------------------------------------------

def test_expert_and_core_ranges_partition_the_layer():
    shape = syn.MoeShape(syn.GLM, 64, 12, 2, 32, 32, 2.5, 1e-5)
    t = quantize_moe_tensors(syn.make_tensors(shape, 5))
    raw, meta = pack_tensors(t)
    lay = MoeLayerLayout.from_meta(meta)
    ranges = lay.routed_expert_ranges()
    core = lay.core_ranges(len(raw))
    assert len(ranges) == 12
    # every routed tensor (weights and scales) lies in its expert's range, nothing else does
    for m in meta:
        a, b = m["offset"], m["offset"] + m["nbytes"]
        if m["name"].startswith("mlp.experts."):
            e = int(m["name"].split(".")[2])
            assert ranges[e][0] <= a and b <= ranges[e][1]
        else:
            assert any(ca <= a and b <= cb for ca, cb in core), m["name"]
    # the pieces tile [0, nbytes) without overlap
    pieces = sorted(ranges + core)
    pos = 0
    for a, b in pieces:
        assert a == pos and b > a
        pos = b
    assert pos == len(raw)
