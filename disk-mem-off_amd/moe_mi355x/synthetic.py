"""Synthetic MoE layers and activations (seeded, reproducible, shape-faithful).

Every tensor draws from its own counter-based stream (``gen.normal``) keyed by
``(seed, crc32(name))``, so a layer can be produced on the host (NumPy) or directly on
the device (``mx_fill_normal``) with the same values.  Distributions follow the
benchmark workloads: activations ~ N(0, 1), weights ~ N(0, 0.02), correction bias
~ N(0, 0.01), RMSNorm weight 1 (or 1 + N(0, 0.1) with ``norm_noise``).
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass

import numpy as np

from . import gen

GLM = "glm4_moe"
QWEN = "qwen3_next"


def stream_of(name: str) -> int:
    return zlib.crc32(name.encode())


@dataclass(frozen=True)
class MoeShape:
    arch: str
    hidden: int
    n_experts: int
    top_k: int
    inter: int
    shared_inter: int
    routed_scaling: float
    eps: float
    has_bias: bool = True
    has_shared_gate: bool = False

    def config(self) -> dict:
        """HF-style config dict with the keys the executors read."""
        cfg = {"hidden_size": self.hidden, "num_experts_per_tok": self.top_k,
               "moe_intermediate_size": self.inter, "norm_topk_prob": True,
               "rms_norm_eps": self.eps, "num_attention_heads": 1}
        if self.arch == GLM:
            cfg.update({"architectures": ["Glm4MoeForCausalLM"], "n_routed_experts": self.n_experts,
                        "routed_scaling_factor": self.routed_scaling, "n_shared_experts": 1,
                        "intermediate_size": self.inter})
        else:
            cfg.update({"architectures": ["Qwen3NextForCausalLM"], "num_experts": self.n_experts,
                        "shared_expert_intermediate_size": self.shared_inter})
        return cfg


# Workload shapes (hidden, experts, top-k, moe_intermediate, shared intermediate).
C1 = MoeShape(GLM, 1024, 16, 4, 256, 256, 2.5, 1e-5)
GLM47 = MoeShape(GLM, 5120, 160, 8, 1536, 1536, 2.5, 1e-5)
QWEN3_NEXT = MoeShape(QWEN, 2048, 512, 10, 512, 512, 1.0, 1e-6, has_bias=False,
                      has_shared_gate=True)


def tensor_specs(shape: MoeShape) -> list[tuple[str, tuple[int, ...], str, float]]:
    """(name, shape, kind, std) for every MoE tensor; kind is 'norm', 'normal' or 'bias'."""
    H, E, I, Is = shape.hidden, shape.n_experts, shape.inter, shape.shared_inter
    specs = [("post_attention_layernorm.weight", (H,), "norm", 0.0),
             ("mlp.gate.weight", (E, H), "normal", 0.02)]
    if shape.has_bias:
        specs.append(("mlp.gate.e_score_correction_bias", (E,), "bias", 0.01))
    for e in range(E):
        specs += [(f"mlp.experts.{e}.gate_proj.weight", (I, H), "normal", 0.02),
                  (f"mlp.experts.{e}.up_proj.weight", (I, H), "normal", 0.02),
                  (f"mlp.experts.{e}.down_proj.weight", (H, I), "normal", 0.02)]
    if Is:
        pre = "mlp.shared_experts." if shape.arch == GLM else "mlp.shared_expert."
        specs += [(pre + "gate_proj.weight", (Is, H), "normal", 0.02),
                  (pre + "up_proj.weight", (Is, H), "normal", 0.02),
                  (pre + "down_proj.weight", (H, Is), "normal", 0.02)]
        if shape.has_shared_gate:
            specs.append(("mlp.shared_expert_gate.weight", (1, H), "normal", 0.02))
    return specs


def make_tensors(shape: MoeShape, seed: int, weight_dtype=np.float32, param_dtype=np.float32,
                 norm_noise: float = 0.0) -> dict[str, np.ndarray]:
    """All MoE tensors of one layer on the host.  Expert weights in ``weight_dtype``
    (float32 / float16), router, bias, norm and shared gate in ``param_dtype``."""
    out = {}
    for name, shp, kind, std in tensor_specs(shape):
        if kind == "norm":
            v = np.ones(shp, dtype=np.float32)
            if norm_noise:
                v = v + gen.normal(seed, stream_of(name), shp, std=norm_noise)
        else:
            v = gen.normal(seed, stream_of(name), shp, std=std)
        is_expert = name.startswith(("mlp.experts.", "mlp.shared_experts.", "mlp.shared_expert."))
        dt = weight_dtype if is_expert else param_dtype
        out[name] = v.astype(dt)
    return out


def make_inputs(seed: int, tokens: int, hidden: int) -> np.ndarray:
    return gen.normal(seed, stream_of("x"), (tokens, hidden), std=1.0)


# ---- Qwen3-Next linear attention (Gated DeltaNet) layers -----------------------------

@dataclass(frozen=True)
class LinearAttnShape:
    """A linear-attention block: ``n_heads`` key heads = value heads (the reference
    reshapes q and k with the value-head count, qwen3_next.py:75-77, 255-258)."""

    hidden: int
    n_heads: int
    head_dim_k: int
    head_dim_v: int
    conv_kernel: int = 4
    eps: float = 1e-6

    @property
    def qkvz_rows(self) -> int:
        return 2 * self.n_heads * (self.head_dim_k + self.head_dim_v)

    @property
    def conv_channels(self) -> int:
        return self.n_heads * (2 * self.head_dim_k + self.head_dim_v)

    @property
    def ba_rows(self) -> int:
        return self.n_heads * (self.head_dim_k + 1)

    def config(self) -> dict:
        """The Qwen3-Next config keys of qwen3_next.py:106-125 for this block."""
        return {"architectures": ["Qwen3NextForCausalLM"], "hidden_size": self.hidden,
                "rms_norm_eps": self.eps, "num_attention_heads": 1,
                "linear_num_key_heads": self.n_heads, "linear_key_head_dim": self.head_dim_k,
                "linear_num_value_heads": self.n_heads,
                "linear_value_head_dim": self.head_dim_v,
                "linear_conv_kernel_dim": self.conv_kernel}


# Qwen3-Next-sized block with as many key heads as value heads (32 x 128).
QWEN3_NEXT_LINEAR = LinearAttnShape(2048, 32, 128, 128, 4, 1e-6)


def linear_attn_specs(shape: LinearAttnShape) -> list[tuple[str, tuple[int, ...], str, float, float]]:
    """(name, shape, kind, std, mean) of every tensor of the block.  Projections
    ~ N(0, 0.02); conv taps ~ N(0, 0.5) (so the conv keeps unit-scale signals);
    A_log ~ N(0, 0.5) and dt_bias ~ N(-4, 0.5), which give per-token decays near 0.95
    (memory of tens of tokens); norm weights 1 (+ noise)."""
    H, n, dk, dv, K = (shape.hidden, shape.n_heads, shape.head_dim_k, shape.head_dim_v,
                       shape.conv_kernel)
    return [("input_layernorm.weight", (H,), "norm", 0.0, 0.0),
            ("linear_attn.in_proj_qkvz.weight", (shape.qkvz_rows, H), "weight", 0.02, 0.0),
            ("linear_attn.in_proj_ba.weight", (shape.ba_rows, H), "weight", 0.02, 0.0),
            ("linear_attn.conv1d.weight", (shape.conv_channels, 1, K), "param", 0.5, 0.0),
            ("linear_attn.A_log", (n,), "param", 0.5, 0.0),
            ("linear_attn.dt_bias", (n,), "param", 0.5, -4.0),
            ("linear_attn.norm.weight", (n * dv,), "norm", 0.0, 0.0),
            ("linear_attn.out_proj.weight", (H, n * dv), "weight", 0.02, 0.0)]


def make_linear_attn_tensors(shape: LinearAttnShape, seed: int, weight_dtype=np.float32,
                             param_dtype=np.float32, norm_noise: float = 0.0
                             ) -> dict[str, np.ndarray]:
    """All tensors of one linear-attention block: projections in ``weight_dtype``, conv
    taps, A_log, dt_bias and norm weights in ``param_dtype``."""
    out = {}
    for name, shp, kind, std, mean in linear_attn_specs(shape):
        if kind == "norm":
            v = np.ones(shp, dtype=np.float32)
            if norm_noise:
                v = v + gen.normal(seed, stream_of(name), shp, std=norm_noise)
        else:
            v = gen.normal(seed, stream_of(name), shp, std=std)
            if mean:
                v = v + np.float32(mean)
        out[name] = v.astype(weight_dtype if kind == "weight" else param_dtype)
    return out


# ---- Qwen3-Next gated full-attention layers --------------------------------------------

@dataclass(frozen=True)
class FullAttnShape:
    """A gated full-attention block (qwen3_next.py:161-205)."""

    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    partial_rotary_factor: float = 0.25
    rope_theta: float = 5000000.0
    eps: float = 1e-6
    qk_norm: bool = True

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)  # qwen3_next.py:118

    def config(self) -> dict:
        """The Qwen3-Next config keys of qwen3_next.py:106-118 for this block."""
        return {"architectures": ["Qwen3NextForCausalLM"], "hidden_size": self.hidden,
                "rms_norm_eps": self.eps, "num_attention_heads": self.n_heads,
                "num_key_value_heads": self.n_kv_heads, "head_dim": self.head_dim,
                "partial_rotary_factor": self.partial_rotary_factor,
                "rope_theta": self.rope_theta}


# Qwen3-Next's full-attention layers: 16 query heads, 2 key/value heads of 256, RoPE on 64.
QWEN3_NEXT_FULL = FullAttnShape(2048, 16, 2, 256, 0.25, 5000000.0, 1e-6)


def full_attn_specs(shape: FullAttnShape) -> list[tuple[str, tuple[int, ...], str, float]]:
    """(name, shape, kind, std): projections ~ N(0, 0.02), norm weights 1 (+ noise)."""
    H, nh, nkv, hd = shape.hidden, shape.n_heads, shape.n_kv_heads, shape.head_dim
    specs = [("input_layernorm.weight", (H,), "norm", 0.0),
             ("self_attn.q_proj.weight", (2 * nh * hd, H), "weight", 0.02),
             ("self_attn.k_proj.weight", (nkv * hd, H), "weight", 0.02),
             ("self_attn.v_proj.weight", (nkv * hd, H), "weight", 0.02),
             ("self_attn.o_proj.weight", (H, nh * hd), "weight", 0.02)]
    if shape.qk_norm:
        specs += [("self_attn.q_norm.weight", (hd,), "norm", 0.0),
                  ("self_attn.k_norm.weight", (hd,), "norm", 0.0)]
    return specs


def make_full_attn_tensors(shape: FullAttnShape, seed: int, weight_dtype=np.float32,
                           param_dtype=np.float32, norm_noise: float = 0.0
                           ) -> dict[str, np.ndarray]:
    """All tensors of one gated full-attention block: projections in ``weight_dtype``,
    norm weights in ``param_dtype``."""
    out = {}
    for name, shp, kind, std in full_attn_specs(shape):
        if kind == "norm":
            v = np.ones(shp, dtype=np.float32)
            if norm_noise:
                v = v + gen.normal(seed, stream_of(name), shp, std=norm_noise)
        else:
            v = gen.normal(seed, stream_of(name), shp, std=std)
        out[name] = v.astype(weight_dtype if kind == "weight" else param_dtype)
    return out
