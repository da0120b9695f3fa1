"""Host dequantizers (KATs of the reference's tests/test_quantize.py:15-113) and the
per-row int8 offline tool."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from moe_mi355x.quantize import (CompositeDequantizer, Float16Dequantizer, Int8Dequantizer,
                                 quantize_moe_tensors)
from moe_mi355x.types import HostBuffer, LayerSpec


def hb(raw: bytes) -> HostBuffer:
    return HostBuffer(view=memoryview(bytearray(raw)), pinned=False)


def test_int8_dequantizer():
    d = Int8Dequantizer()
    assert d.needs_dequantize(LayerSpec(0, "L", 4, {"dtype": "int8"}))
    assert not d.needs_dequantize(LayerSpec(0, "L", 4))
    assert not d.needs_dequantize(LayerSpec(0, "L", 4, {"dtype": "float16"}))
    assert d.decompressed_nbytes(LayerSpec(0, "L", 100, {"dtype": "int8"})) == 400
    out = d.dequantize(LayerSpec(0, "L", 2, {"dtype": "int8", "scale": 0.5}), hb(struct.pack("2b", 4, -2)))
    assert struct.unpack("2f", out.view.tobytes()) == pytest.approx((2.0, -1.0))
    out = d.dequantize(LayerSpec(0, "L", 1, {"dtype": "int8", "zero_point": 10}), hb(struct.pack("1b", 15)))
    assert struct.unpack("1f", out.view.tobytes())[0] == pytest.approx(5.0)
    assert d.dequantize(LayerSpec(0, "L", 4, {"dtype": "int8"}), hb(b"\x01\x02\x03\x04")).nbytes == 16


def test_float16_dequantizer():
    d = Float16Dequantizer()
    assert d.needs_dequantize(LayerSpec(0, "L", 4, {"dtype": "float16"}))
    assert d.decompressed_nbytes(LayerSpec(0, "L", 8, {"dtype": "float16"})) == 16
    out = d.dequantize(LayerSpec(0, "L", 4, {"dtype": "float16"}), hb(struct.pack("2e", 1.0, 2.0)))
    assert out.nbytes == 8 and struct.unpack("2f", out.view.tobytes()) == pytest.approx((1.0, 2.0))


def test_composite_dequantizer():
    d = CompositeDequantizer()
    assert d.decompressed_nbytes(LayerSpec(0, "L", 4, {"dtype": "int8"})) == 16
    assert d.decompressed_nbytes(LayerSpec(0, "L", 4, {"dtype": "float16"})) == 8
    plain = LayerSpec(0, "L", 16)
    buf = hb(bytes(16))
    assert not d.needs_dequantize(plain) and d.dequantize(plain, buf) is buf
    out = d.dequantize(LayerSpec(0, "L", 2, {"dtype": "int8", "scale": 2.0}), hb(struct.pack("2b", 3, -1)))
    assert struct.unpack("2f", out.view.tobytes()) == pytest.approx((6.0, -2.0))


def test_quantize_moe_tensors_only_touches_expert_projections():
    rng = np.random.default_rng(0)
    t = {"mlp.gate.weight": rng.standard_normal((4, 8)).astype(np.float32),
         "mlp.experts.0.gate_proj.weight": rng.standard_normal((6, 8)).astype(np.float32),
         "mlp.shared_expert.down_proj.weight": rng.standard_normal((8, 6)).astype(np.float32),
         "mlp.shared_expert_gate.weight": rng.standard_normal((1, 8)).astype(np.float32)}
    q = quantize_moe_tensors(t)
    assert q["mlp.gate.weight"].dtype == np.float32
    assert q["mlp.shared_expert_gate.weight"].dtype == np.float32
    assert q["mlp.experts.0.gate_proj.weight"].dtype == np.int8
    assert q["mlp.experts.0.gate_proj.weight_scale"].shape == (6,)
    assert q["mlp.shared_expert.down_proj.weight_scale"].dtype == np.float16
