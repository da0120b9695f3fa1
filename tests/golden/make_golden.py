"""Write golden vectors of the reference MoE block (run in the build container only).

The end-to-end output of ``GLM4MoeExecutor._moe_mlp_block``
(offload_runtime/executors/glm4_moe.py:176-240) and ``Qwen3NextExecutor._moe_mlp_block``
(offload_runtime/executors/qwen3_next.py:273-333) is not pinned by any test of the
reference (its integration tests check shapes and finiteness only), so this script runs
the reference executors from a local checkout on seeded synthetic inputs and stores
their outputs.  Inputs are not stored: they are regenerated from (shape, seed) by
``moe_mi355x.synthetic`` and checked against the stored SHA-256 digests.

Usage:  python tests/golden/make_golden.py /path/to/disk-mem-off
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "disk-mem-off_amd"))

from moe_mi355x import synthetic as syn  # noqa: E402

CASES = [
    # name, shape, seed, tokens, compute dtype, norm noise
    ("glm_c1_f32", syn.C1, 1234, 8, "float32", 0.0),
    ("glm_c1_f16", syn.C1, 1234, 8, "float16", 0.0),
    ("glm_c1_f32_norm", syn.C1, 77, 8, "float32", 0.1),
    ("glm_tiny_f32", syn.MoeShape(syn.GLM, 8, 4, 2, 8, 8, 1.0, 1e-6), 789, 3, "float32", 0.0),
    ("qwen_small_f32", syn.MoeShape(syn.QWEN, 512, 32, 4, 128, 128, 1.0, 1e-6, has_bias=False,
                                    has_shared_gate=True), 4321, 8, "float32", 0.0),
    ("qwen_tiny_f32", syn.MoeShape(syn.QWEN, 8, 4, 2, 4, 4, 1.0, 1e-6, has_bias=False,
                                   has_shared_gate=True), 999, 3, "float32", 0.0),
]


def digest(arrays: dict[str, np.ndarray]) -> str:
    h = hashlib.sha256()
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        h.update(name.encode())
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def case_inputs(shape: syn.MoeShape, seed: int, tokens: int, dtype: str, norm_noise: float):
    dt = np.dtype(dtype)
    t = syn.make_tensors(shape, seed, weight_dtype=dt, param_dtype=dt, norm_noise=norm_noise)
    x = syn.make_inputs(seed, tokens, shape.hidden)
    return x, t


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from offload_runtime.executors.glm4_moe import GLM4MoeExecutor
    from offload_runtime.executors.qwen3_next import Qwen3NextExecutor

    index = {}
    for name, shape, seed, tokens, dtype, noise in CASES:
        x, t = case_inputs(shape, seed, tokens, dtype, noise)
        cfg = shape.config()
        ex = GLM4MoeExecutor(cfg) if shape.arch == syn.GLM else Qwen3NextExecutor(cfg)
        out = ex._moe_mlp_block(x, t)
        np.savez(HERE / f"{name}.npz", out=np.asarray(out, dtype=np.float32))
        index[name] = {"arch": shape.arch, "hidden": shape.hidden, "n_experts": shape.n_experts,
                       "top_k": shape.top_k, "inter": shape.inter,
                       "shared_inter": shape.shared_inter, "routed_scaling": shape.routed_scaling,
                       "eps": shape.eps, "has_bias": shape.has_bias,
                       "has_shared_gate": shape.has_shared_gate, "seed": seed, "tokens": tokens,
                       "dtype": dtype, "norm_noise": noise, "x_sha256": digest({"x": x}),
                       "tensors_sha256": digest(t)}
        print(f"{name}: out[0,:4]={np.asarray(out)[0, :4]}")
    (HERE / "index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
