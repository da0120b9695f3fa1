"""The offline per-row int8 quantiser over a safetensors checkpoint (CPU only)."""
from __future__ import annotations

import json

import numpy as np
import pytest

from moe_mi355x import _lib, synthetic as syn
from moe_mi355x.layout import MoeLayerLayout, unpack_host
from moe_mi355x.quantize import dequantize_rows_int8, quantize_rows_int8
from moe_mi355x.quantize_tool import load_layer, main, quantize_checkpoint

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")


def _write_checkpoint(d, shape):
    t = syn.make_tensors(shape, 11, weight_dtype=np.float16)
    full = {f"model.layers.0.{n}": v for n, v in t.items()}
    full["model.embed_tokens.weight"] = np.ones((4, shape.hidden), np.float32)
    names = sorted(full)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half],
              "model-00002-of-00002.safetensors": names[half:]}
    weight_map = {}
    for fname, ns in shards.items():
        tens = {n: torch.from_numpy(np.ascontiguousarray(full[n])) for n in ns}
        # one bf16 expert matrix, as real checkpoints store them
        for n in ns:
            if n.endswith("experts.1.up_proj.weight"):
                tens[n] = tens[n].to(torch.bfloat16)
        st_torch.save_file(tens, str(d / fname))
        weight_map.update({n: fname for n in ns})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    (d / "config.json").write_text(json.dumps({"hidden_size": shape.hidden}))
    return full


def test_quantize_checkpoint(tmp_path):
    shape = syn.MoeShape(syn.GLM, 64, 4, 2, 32, 32, 2.5, 1e-5)
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    full = _write_checkpoint(src, shape)
    assert main([str(src), str(dst)]) == 0
    out = {}
    for f in sorted(dst.glob("*.safetensors")):
        out.update({k: v for k, v in st_torch.load_file(str(f)).items()})
    idx = json.loads((dst / "model.safetensors.index.json").read_text())["weight_map"]
    assert (dst / "config.json").exists()
    n_expert_mats = 3 * (shape.n_experts + 1)
    scales = [n for n in out if n.endswith("_scale")]
    assert len(scales) == n_expert_mats and all(n in idx for n in scales)
    for name, src_arr in full.items():
        got = out[name]
        if name.endswith("_proj.weight") and ".mlp." in name:
            assert got.dtype == torch.int8
            w = src_arr.astype(np.float32)
            if name.endswith("experts.1.up_proj.weight"):  # stored bf16 in the source
                w = torch.from_numpy(src_arr).to(torch.bfloat16).to(torch.float32).numpy()
            q, s = quantize_rows_int8(w)
            assert np.array_equal(got.numpy(), q)
            assert np.array_equal(out[name + "_scale"].numpy(), s)
            deq = dequantize_rows_int8(got.numpy(), out[name + "_scale"].numpy())
            assert np.max(np.abs(deq - w)) <= 0.51 * float(np.max(s.astype(np.float32)))
        else:
            assert np.array_equal(got.numpy(), src_arr)
    # the layer read back from the output is a per-row int8 MoE layer with the same bytes
    buf, meta = load_layer(dst, 0)
    lay = MoeLayerLayout.from_meta(meta)
    assert lay.n_experts == shape.n_experts and lay.shared_inter == shape.shared_inter
    assert lay.weight_dtype == _lib.MX_DT_I8
    views = unpack_host(bytes(buf), meta)
    for name, arr in views.items():
        want = out["model.layers.0." + name]
        if want.dtype == torch.bfloat16:
            want = want.to(torch.float32)
        assert np.array_equal(arr, want.numpy()), name
    with pytest.raises(KeyError):
        load_layer(dst, 7)


def test_quantize_checkpoint_rejects_empty_dir(tmp_path):
    with pytest.raises(ValueError, match="no .safetensors"):
        quantize_checkpoint(tmp_path, tmp_path / "out")
