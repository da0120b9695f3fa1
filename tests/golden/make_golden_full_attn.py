"""Write golden vectors of the reference gated full-attention block (build container only).

The composed output of ``Qwen3NextExecutor._full_attn_block``
(offload_runtime/executors/qwen3_next.py:161-205) — which half of q_proj is the gate, the
head layout, the qk-norm and partial-RoPE order, GQA repetition, the causal mask — is pinned
by no test of the reference (its integration test checks shapes and finiteness), so this
script runs that method from a local checkout on seeded synthetic inputs and stores the
outputs.  Inputs are regenerated from (shape, seed) by ``moe_mi355x.synthetic`` and checked
against the stored SHA-256 digests.

Usage:  python tests/golden/make_golden_full_attn.py /path/to/disk-mem-off
"""
from __future__ import annotations

import dataclasses
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "disk-mem-off_amd"))

from moe_mi355x import synthetic as syn  # noqa: E402
from make_golden import digest  # noqa: E402

CASES = [
    # name, shape, seed, tokens, dtype, norm noise
    ("fa_tiny_f32", syn.FullAttnShape(8, 2, 1, 4, 0.5, 5000000.0, 1e-6), 999, 3, "float32", 0.0),
    ("fa_small_f32", syn.FullAttnShape(64, 4, 2, 16, 0.25, 10000.0, 1e-6), 41, 37, "float32", 0.1),
    ("fa_full_rope_f32", syn.FullAttnShape(64, 2, 2, 32, 1.0, 10000.0, 1e-5), 42, 19, "float32",
     0.1),
    ("fa_mid_f32", syn.FullAttnShape(256, 8, 2, 64, 0.25, 5000000.0, 1e-6), 43, 70, "float32",
     0.1),
    ("fa_mid_f16", syn.FullAttnShape(256, 8, 2, 64, 0.25, 5000000.0, 1e-6), 44, 33, "float16",
     0.0),
    ("fa_nonorm_f32", syn.FullAttnShape(64, 4, 4, 16, 0.5, 10000.0, 1e-6, qk_norm=False), 45, 11,
     "float32", 0.0),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from offload_runtime.executors.qwen3_next import Qwen3NextExecutor

    index = {}
    for name, shape, seed, tokens, dtype, noise in CASES:
        dt = np.dtype(dtype)
        t = syn.make_full_attn_tensors(shape, seed, weight_dtype=dt, param_dtype=dt,
                                       norm_noise=noise)
        x = syn.make_inputs(seed, tokens, shape.hidden)
        ex = Qwen3NextExecutor(shape.config())
        out = np.asarray(ex._full_attn_block(x, t), dtype=np.float32)
        np.savez(HERE / f"{name}.npz", out=out)
        index[name] = {"shape": dataclasses.asdict(shape), "seed": seed, "tokens": tokens,
                       "dtype": dtype, "norm_noise": noise, "x_sha256": digest({"x": x}),
                       "tensors_sha256": digest(t)}
        print(f"{name}: out[0,:4]={out[0, :4]}")
    (HERE / "full_attn_index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
