"""Packed MoE layer buffers: packing, metadata parsing, device pointer tables.

The layer buffer contract is the one the reference loader emits for MoE layers
(offload_runtime/loader/huggingface.py:458-591): every tensor of the layer is packed
contiguously in lexicographic order of its short name, and ``LayerSpec.metadata["tensors"]``
lists ``{name, shape, dtype, offset, nbytes}`` (read back by ``_unpack_tensors``,
offload_runtime/executors/_common.py:43-58).  The executors here never read the buffer
back: they turn the offsets into device addresses inside ``DeviceBuffer.handle``.

Tensor names (GLM4-MoE, glm4_moe.py:48-60; Qwen3-Next, qwen3_next.py:278-328):
  post_attention_layernorm.weight                       [H]
  mlp.gate.weight                                       [E, H]
  mlp.gate.e_score_correction_bias                      [E]      (GLM, optional)
  mlp.experts.{e}.{gate,up}_proj.weight                 [I, H]
  mlp.experts.{e}.down_proj.weight                      [H, I]
  mlp.shared_experts.{gate,up,down}_proj.weight         (GLM, optional)
  mlp.shared_expert.{gate,up,down}_proj.weight          (Qwen3-Next, optional)
  mlp.shared_expert_gate.weight                         [1, H]   (Qwen3-Next, optional)
Per-row int8 experts add ``<name>_scale`` (fp16, one per output row) next to each int8
``<name>`` (``...proj.weight`` -> ``...proj.weight_scale``).
"""
from __future__ import annotations

import ctypes
import re
from dataclasses import dataclass, field
from typing import Any

import numpy as np

from . import _lib
from .types import LayerSpec

NORM = "post_attention_layernorm.weight"
ROUTER = "mlp.gate.weight"
BIAS = "mlp.gate.e_score_correction_bias"
SHARED_GATE = "mlp.shared_expert_gate.weight"
SHARED_PREFIXES = ("mlp.shared_experts.", "mlp.shared_expert.")
PROJ = ("gate_proj", "up_proj", "down_proj")
_EXPERT_RE = re.compile(r"^mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight(_scale)?$")

_DT_CODES = {"float32": _lib.MX_DT_F32, "float16": _lib.MX_DT_F16, "int8": _lib.MX_DT_I8}


def pack_tensors(tensors: dict[str, np.ndarray], align: int = 1,
                 order: list[str] | None = None) -> tuple[bytearray, list[dict[str, Any]]]:
    """Pack arrays into one buffer (lexicographic name order unless ``order`` is given).

    ``align = 1`` reproduces the loader's contiguous packing; a larger value pads each
    tensor's offset to that many bytes.
    """
    names = order if order is not None else sorted(tensors)
    meta: list[dict[str, Any]] = []
    offset = 0
    for name in names:
        arr = np.ascontiguousarray(tensors[name])
        offset = (offset + align - 1) // align * align
        meta.append({"name": name, "shape": list(arr.shape), "dtype": arr.dtype.name,
                     "offset": offset, "nbytes": arr.nbytes})
        offset += arr.nbytes
    buf = bytearray(offset)
    for m in meta:
        arr = np.ascontiguousarray(tensors[m["name"]])
        buf[m["offset"]: m["offset"] + m["nbytes"]] = arr.tobytes()
    return buf, meta


def make_layer_spec(layer_id: int, meta: list[dict[str, Any]], nbytes: int,
                    **extra: Any) -> LayerSpec:
    md = {"tensors": meta, "full_prefix": f"model.layers.{layer_id}.", "is_moe": True}
    md.update(extra)
    return LayerSpec(layer_id=layer_id, name=f"model.layers.{layer_id}", nbytes=nbytes,
                     metadata=md)


def unpack_host(raw: Any, meta: list[dict[str, Any]]) -> dict[str, np.ndarray]:
    """Zero-copy NumPy views of a packed host buffer (host side of _common.py:43-58)."""
    out = {}
    for m in meta:
        dt = np.dtype(m["dtype"])
        arr = np.frombuffer(raw, dtype=dt, count=m["nbytes"] // dt.itemsize, offset=m["offset"])
        out[m["name"]] = arr.reshape(m["shape"])
    return out


def rows_to_frag16(mat: np.ndarray) -> np.ndarray:
    """Row-major [rows, cols] -> MX_LAYOUT_FRAG16 bytes: 1 KiB per (16 rows, 64 bytes of
    columns) fragment, fragments column-block-minor, lane 16 q + j of a fragment holding
    bytes 16 q .. 16 q + 15 of the fragment's row j (the device converter's layout)."""
    rows = mat.shape[0]
    b = np.ascontiguousarray(mat).view(np.uint8).reshape(rows, -1)
    nch = b.shape[1] // 64
    if rows % 16 or b.shape[1] % 64:
        raise ValueError("no whole fragments")
    return np.ascontiguousarray(
        b.reshape(rows // 16, 16, nch, 4, 16).transpose(0, 2, 3, 1, 4)).reshape(-1)


def frag16_to_rows(buf: np.ndarray, rows: int, cols: int, dtype: Any) -> np.ndarray:
    """Inverse of ``rows_to_frag16``."""
    esz = np.dtype(dtype).itemsize
    nch = cols * esz // 64
    b = np.ascontiguousarray(buf).view(np.uint8).reshape(rows // 16, nch, 4, 16, 16)
    return np.ascontiguousarray(b.transpose(0, 3, 1, 2, 4)).reshape(rows, cols * esz).view(dtype)


@dataclass
class MoeLayerLayout:
    """Where each MoE tensor lives inside a packed layer buffer, with derived shapes."""

    hidden: int
    inter: int
    shared_inter: int
    n_experts: int
    weight_dtype: int
    param_dtype: int
    entries: dict[str, dict[str, Any]] = field(repr=False)
    shared_prefix: str | None = None
    has_bias: bool = False
    has_shared_gate: bool = False

    @classmethod
    def from_meta(cls, meta: list[dict[str, Any]]) -> "MoeLayerLayout":
        entries = {m["name"]: m for m in meta}
        for req in (NORM, ROUTER):
            if req not in entries:
                raise ValueError(f"MoE layer is missing tensor {req!r}")
        E, H = entries[ROUTER]["shape"]
        experts: dict[int, dict[str, dict[str, Any]]] = {}
        for name, m in entries.items():
            mt = _EXPERT_RE.match(name)
            if mt:
                experts.setdefault(int(mt.group(1)), {})[mt.group(2) + (mt.group(3) or "")] = m
        if sorted(experts) != list(range(E)):
            raise ValueError(f"expected experts 0..{E - 1}, found {len(experts)} expert ids")
        e0 = experts[0]
        wdt_name = e0["gate_proj"]["dtype"]
        if wdt_name not in _DT_CODES:
            raise ValueError(f"unsupported expert weight dtype {wdt_name}")
        I = e0["gate_proj"]["shape"][0]
        for e, d in experts.items():
            for p in PROJ:
                if p not in d:
                    raise ValueError(f"expert {e} is missing {p}")
                if d[p]["dtype"] != wdt_name:
                    raise ValueError("all expert weights must share one dtype")
                if wdt_name == "int8" and p + "_scale" not in d:
                    raise ValueError(f"int8 expert {e} {p} has no per-row scale tensor")
            if d["gate_proj"]["shape"] != [I, H] or d["up_proj"]["shape"] != [I, H] or \
                    d["down_proj"]["shape"] != [H, I]:
                raise ValueError(f"expert {e} has inconsistent shapes")
        shared_prefix = None
        Is = 0
        for pre in SHARED_PREFIXES:
            if pre + "gate_proj.weight" in entries:
                shared_prefix = pre
                Is = entries[pre + "gate_proj.weight"]["shape"][0]
                for p in PROJ:
                    m = entries.get(pre + p + ".weight")
                    if m is None or m["dtype"] != wdt_name:
                        raise ValueError(f"shared expert {p} missing or of another dtype")
                    if wdt_name == "int8" and pre + p + ".weight_scale" not in entries:
                        raise ValueError(f"int8 shared expert {p} has no scale tensor")
                if entries[pre + "down_proj.weight"]["shape"] != [H, Is]:
                    raise ValueError("shared expert down_proj has an inconsistent shape")
                break
        pdt_name = entries[ROUTER]["dtype"]
        params = [NORM, ROUTER] + [n for n in (BIAS, SHARED_GATE) if n in entries]
        for n in params:
            if entries[n]["dtype"] != pdt_name:
                raise ValueError("norm / router / bias / shared gate must share one dtype")
        if pdt_name not in ("float32", "float16"):
            raise ValueError(f"unsupported parameter dtype {pdt_name}")
        lay = cls(hidden=H, inter=I, shared_inter=Is, n_experts=E,
                  weight_dtype=_DT_CODES[wdt_name], param_dtype=_DT_CODES[pdt_name],
                  entries=entries, shared_prefix=shared_prefix, has_bias=BIAS in entries,
                  has_shared_gate=SHARED_GATE in entries and shared_prefix is not None)
        lay._experts = experts
        return lay

    def offset(self, name: str) -> int:
        return int(self.entries[name]["offset"])

    def expert_offsets(self) -> list[tuple[int, int, int, int, int, int]]:
        """(gate, up, down, gate_scale, up_scale, down_scale) byte offsets, shared last;
        -1 marks an absent tensor."""
        rows = []
        for e in range(self.n_experts):
            d = self._experts[e]
            rows.append(tuple(int(d[p]["offset"]) for p in PROJ) +
                        tuple(int(d[p + "_scale"]["offset"]) if p + "_scale" in d else -1
                              for p in PROJ))
        if self.shared_prefix:
            pre = self.shared_prefix
            rows.append(tuple(self.offset(pre + p + ".weight") for p in PROJ) +
                        tuple(self.offset(pre + p + ".weight_scale")
                              if pre + p + ".weight_scale" in self.entries else -1
                              for p in PROJ))
        else:
            rows.append((-1,) * 6)
        return rows

    def routed_expert_ranges(self) -> list[tuple[int, int]]:
        """Byte range [start, end) of each routed expert's tensors (weights and scales);
        the loader's lexicographic packing keeps each expert's tensors adjacent."""
        out = []
        for e in range(self.n_experts):
            ms = self._experts[e].values()
            out.append((min(int(m["offset"]) for m in ms),
                        max(int(m["offset"]) + int(m["nbytes"]) for m in ms)))
        return out

    def core_ranges(self, total: int) -> list[tuple[int, int]]:
        """Byte ranges of [0, total) outside every routed expert: norms, router, bias,
        shared expert(s), any other tensor of the layer, and padding."""
        out, pos = [], 0
        for a, b in sorted(self.routed_expert_ranges()):
            if a > pos:
                out.append((pos, a))
            pos = max(pos, b)
        if pos < total:
            out.append((pos, total))
        return out

    def expert_matrices(self) -> list[tuple[int, int, int]]:
        """(byte offset, rows, cols) of every expert weight matrix, shared expert last."""
        out = []
        for offs in self.expert_offsets():
            if offs[0] < 0:
                continue
            shared = len(out) >= 3 * self.n_experts
            inter = self.shared_inter if shared else self.inter
            out += [(offs[0], inter, self.hidden), (offs[1], inter, self.hidden),
                    (offs[2], self.hidden, inter)]
        return out

    def expert_table(self, base: int) -> ctypes.Array:
        """Device pointer table (E + 1 ``MxExpertPtrs``) for a buffer at address ``base``.

        Raises ``ValueError`` when a weight is not 16-byte aligned (the kernels stream
        weights in 16-byte pieces)."""
        table = (_lib.MxExpertPtrs * (self.n_experts + 1))()
        for i, offs in enumerate(self.expert_offsets()):
            ptrs = [base + o if o >= 0 else 0 for o in offs]
            for p, o in zip(ptrs[:3], offs[:3]):
                if o >= 0 and p % 16:
                    raise ValueError(
                        f"expert weight at offset {o} is not 16-byte aligned; repack the layer "
                        "with pack_tensors(align=16) or larger")
            table[i] = _lib.MxExpertPtrs(*[p or None for p in ptrs])
        return table

    def weights(self, base: int, table_dev: int) -> _lib.MxMoeWeights:
        def addr(name: str) -> int | None:
            return base + self.offset(name) if name in self.entries else None
        return _lib.MxMoeWeights(
            norm_w=addr(NORM), router_w=addr(ROUTER),
            bias=addr(BIAS) if self.has_bias else None,
            shared_gate_w=addr(SHARED_GATE) if self.has_shared_gate else None,
            experts=table_dev)
