"""Offline per-row int8 quantiser for safetensors checkpoints.

    python -m moe_mi355x.quantize_tool <checkpoint dir or .safetensors file> <output dir>

Every routed / shared expert projection ``...mlp.experts.<e>.<proj>.weight`` and
``...mlp.shared_expert(s).<proj>.weight`` (2-D; fp32, fp16 or bf16) becomes an int8 tensor
of the same name plus ``<name>_scale`` (fp16, one per output row), by the rule of
``quantize.quantize_rows_int8``; every other tensor is copied unchanged.  Shard files keep
their names; ``model.safetensors.index.json`` gets the scale tensors added to its weight
map, and the other ``*.json`` files are copied.

``load_layer`` reads one decoder layer back from such a checkpoint, keeping each tensor's
stored type (int8 weights, fp16 scales; bf16 becomes fp32), and packs it in lexicographic
name order: the per-row int8 layer the expert kernels read directly (no host
dequantisation: leave ``metadata["dtype"]`` unset).  The reference loader casts every tensor
to one compute dtype (loader/huggingface.py:611-618), which would expand the int8 weights.

The reference stores quantised layers only as a whole-layer int8 block with one scalar
scale (offload_runtime/quantize.py:14-50); this is the per-row on-disk form of that scheme.
"""
from __future__ import annotations

import json
import re
import shutil
import sys
from pathlib import Path

import numpy as np

from .quantize import quantize_rows_int8

_EXPERT_W = re.compile(r"(^|\.)mlp\.(experts\.\d+|shared_experts?)\.(gate|up|down)_proj\.weight$")


def _load(path: Path) -> dict:
    import safetensors.torch

    return safetensors.torch.load_file(str(path))


def quantize_file(src: Path, dst: Path) -> list[str]:
    """Quantise one shard; returns the names of the scale tensors it added."""
    import safetensors.torch
    import torch

    tensors = _load(src)
    out: dict = {}
    added: list[str] = []
    for name in sorted(tensors):
        t = tensors[name]
        if _EXPERT_W.search(name) and t.dim() == 2:
            q, s = quantize_rows_int8(t.to(torch.float32).numpy())
            out[name] = torch.from_numpy(q)
            out[name + "_scale"] = torch.from_numpy(s)
            added.append(name + "_scale")
        else:
            out[name] = t
    dst.parent.mkdir(parents=True, exist_ok=True)
    safetensors.torch.save_file(out, str(dst), metadata={"format": "pt"})
    return added


def quantize_checkpoint(src: Path, dst: Path) -> dict[str, int]:
    """Quantise a checkpoint directory (or one file); returns counts of what was written."""
    src, dst = Path(src), Path(dst)
    files = [src] if src.is_file() else sorted(src.glob("*.safetensors"))
    if not files:
        raise ValueError(f"no .safetensors files under {src}")
    dst.mkdir(parents=True, exist_ok=True)
    weight_map: dict[str, str] = {}
    n_scales = 0
    for f in files:
        added = quantize_file(f, dst / f.name)
        n_scales += len(added)
        for a in added:
            weight_map[a] = f.name
    if src.is_dir():
        for j in src.glob("*.json"):
            if j.name == "model.safetensors.index.json":
                idx = json.loads(j.read_text())
                idx.setdefault("weight_map", {}).update(weight_map)
                (dst / j.name).write_text(json.dumps(idx, indent=2))
            else:
                shutil.copy2(j, dst / j.name)
    return {"files": len(files), "scales": n_scales}


def load_layer(ckpt: Path, layer_id: int, align: int = 16) -> tuple[bytearray, list[dict]]:
    """Pack ``model.layers.<layer_id>.*`` of a checkpoint directory (or file) for upload.

    Returns the packed bytes and the tensor metadata that ``layout.make_layer_spec`` and
    ``layout.MoeLayerLayout.from_meta`` take.
    """
    import torch
    from safetensors import safe_open

    from .layout import pack_tensors

    ckpt = Path(ckpt)
    files = [ckpt] if ckpt.is_file() else sorted(ckpt.glob("*.safetensors"))
    prefix = f"model.layers.{layer_id}."
    tensors: dict[str, np.ndarray] = {}
    for f in files:
        with safe_open(str(f), framework="pt") as h:
            for name in h.keys():
                if not name.startswith(prefix):
                    continue
                t = h.get_tensor(name)
                if t.dtype == torch.bfloat16:
                    t = t.to(torch.float32)
                tensors[name[len(prefix):]] = t.numpy()
    if not tensors:
        raise KeyError(f"no tensors under {prefix!r} in {ckpt}")
    return pack_tensors(tensors, align=align)


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 2:
        print(__doc__.split("\n\n")[1], file=sys.stderr)
        return 2
    res = quantize_checkpoint(Path(argv[0]), Path(argv[1]))
    print(f"quantised {res['scales']} expert matrices in {res['files']} file(s) -> {argv[1]}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
