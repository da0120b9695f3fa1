"""ctypes bindings of ``libmoe_mi355x.so`` (declared in ``include/moe_mi355x.h``).

The library is the only compute path: there is no NumPy or PyTorch fallback.  Loading
fails loudly (``RuntimeError``) when the shared library has not been built.

Status convention (mirrors ``_check`` in offload_runtime/backends/rocm_backend.py:15-24):
a positive HIP status becomes ``RuntimeError("HIP runtime call failed with status=N")``;
argument errors detected by the library become ``ValueError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmoe_mi355x.so"

MX_OK = 0
MX_ERR_INVALID = -1
MX_ERR_UNSUPPORTED = -2
MX_ERR_WORKSPACE = -3
MX_ERR_ALIGNMENT = -4

MX_DT_F32 = 0
MX_DT_F16 = 1
MX_DT_I8 = 2

MX_ROUTER_REF_SOFTMAX_BIAS = 0
MX_ROUTER_SIGMOID_SELECT_BIAS = 1
MX_ROUTER_SOFTMAX = 2
MX_STAGE_ROUTE_END = 4
MX_LAYOUT_ROWS = 0
MX_LAYOUT_FRAG16 = 1

MX_N_STAGES = 7
MX_NOALLOC_MAX_WORKSPACE = 16 << 20
STAGE_NAMES = ("rmsnorm", "router_logits", "router_topk", "dispatch", "expert_gate_up",
               "expert_down", "combine")

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_size_t = ctypes.c_size_t
c_float = ctypes.c_float
c_uint64 = ctypes.c_uint64


class MxExpertPtrs(ctypes.Structure):
    _fields_ = [("gate", c_void_p), ("up", c_void_p), ("down", c_void_p),
                ("gate_scale", c_void_p), ("up_scale", c_void_p), ("down_scale", c_void_p)]


class MxMoeDesc(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int32), ("inter", c_int32), ("shared_inter", c_int32),
        ("n_experts", c_int32), ("top_k", c_int32), ("router_mode", c_int32),
        ("norm_topk_prob", c_int32), ("weight_dtype", c_int32), ("param_dtype", c_int32),
        ("has_bias", c_int32), ("has_shared_gate", c_int32),
        ("routed_scaling", c_float), ("eps", c_float), ("weight_layout", c_int32),
    ]


class MxMoeWeights(ctypes.Structure):
    _fields_ = [("norm_w", c_void_p), ("router_w", c_void_p), ("bias", c_void_p),
                ("shared_gate_w", c_void_p), ("experts", c_void_p)]


class MxMoeViews(ctypes.Structure):
    _fields_ = [
        ("h32", c_void_p), ("h16", c_void_p), ("logits", c_void_p), ("router_splits", c_int32),
        ("topk_ids", c_void_p), ("topk_w", c_void_p), ("shared_w", c_void_p),
        ("counts", c_void_p), ("offsets", c_void_p), ("sorted_tok", c_void_p),
        ("sorted_w", c_void_p), ("pair_pos", c_void_p), ("g_expert", c_void_p),
        ("g_start", c_void_p), ("g_count", c_void_p), ("n_groups", c_void_p),
        ("mt_group", c_void_p), ("mt_row0", c_void_p), ("n_mtiles", c_void_p),
        ("m_blk", c_int32), ("act", c_void_p), ("y", c_void_p),
    ]


MX_LA_N_STAGES = 8
LA_STAGE_NAMES = ("rmsnorm", "qkvz_proj", "ba_proj", "conv_gates", "scan", "gated_norm",
                  "out_proj", "residual")


class MxLinearAttnDesc(ctypes.Structure):
    _fields_ = [("hidden", c_int32), ("n_heads", c_int32), ("head_dim_k", c_int32),
                ("head_dim_v", c_int32), ("conv_kernel", c_int32), ("weight_dtype", c_int32),
                ("param_dtype", c_int32), ("eps", c_float)]


class MxLinearAttnWeights(ctypes.Structure):
    _fields_ = [("norm_w", c_void_p), ("qkvz_w", c_void_p), ("qkvz_scale", c_void_p),
                ("ba_w", c_void_p), ("ba_scale", c_void_p), ("conv_w", c_void_p),
                ("a_log", c_void_p), ("dt_bias", c_void_p), ("out_norm_w", c_void_p),
                ("out_w", c_void_p), ("out_scale", c_void_p)]


class MxLinearAttnViews(ctypes.Structure):
    _fields_ = [("h32", c_void_p), ("h16", c_void_p), ("qkvz", c_void_p), ("ba", c_void_p),
                ("q", c_void_p), ("kb", c_void_p), ("v", c_void_p), ("decay", c_void_p),
                ("o", c_void_p), ("act", c_void_p), ("y", c_void_p)]


MX_FA_N_STAGES = 8
FA_STAGE_NAMES = ("rmsnorm", "q_proj", "k_proj", "v_proj", "qk_rope", "attention", "o_proj",
                  "residual")


class MxFullAttnDesc(ctypes.Structure):
    _fields_ = [("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
                ("head_dim", c_int32), ("rotary_dim", c_int32), ("weight_dtype", c_int32),
                ("param_dtype", c_int32), ("rope_theta", ctypes.c_double), ("eps", c_float)]


class MxFullAttnWeights(ctypes.Structure):
    _fields_ = [("norm_w", c_void_p), ("q_w", c_void_p), ("q_scale", c_void_p),
                ("k_w", c_void_p), ("k_scale", c_void_p), ("v_w", c_void_p),
                ("v_scale", c_void_p), ("o_w", c_void_p), ("o_scale", c_void_p),
                ("q_norm_w", c_void_p), ("k_norm_w", c_void_p)]


class MxFullAttnViews(ctypes.Structure):
    _fields_ = [("h32", c_void_p), ("h16", c_void_p), ("qg", c_void_p), ("k", c_void_p),
                ("v", c_void_p), ("act", c_void_p), ("y", c_void_p)]


class MxDeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("cu_count", c_int32), ("clock_khz", c_int32), ("mem_clock_khz", c_int32),
                ("mem_bus_width", c_int32), ("total_mem", ctypes.c_int64),
                ("l2_bytes", c_int32), ("lds_per_block", c_int32)]


P = ctypes.POINTER
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mx_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mx_get_device_count": (ctypes.c_int, [P(c_int32)]),
    "mx_device_info": (ctypes.c_int, [c_int32, P(MxDeviceInfo)]),
    "mx_set_device": (ctypes.c_int, [c_int32]),
    "mx_device_sync": (ctypes.c_int, []),
    "mx_malloc": (ctypes.c_int, [P(c_void_p), c_size_t]),
    "mx_free": (ctypes.c_int, [c_void_p]),
    "mx_host_malloc": (ctypes.c_int, [P(c_void_p), c_size_t]),
    "mx_host_free": (ctypes.c_int, [c_void_p]),
    "mx_memcpy_h2d_async": (ctypes.c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "mx_memcpy_d2h_async": (ctypes.c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "mx_memcpy_d2d_async": (ctypes.c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "mx_stream_create": (ctypes.c_int, [P(c_void_p), c_int32]),
    "mx_stream_destroy": (ctypes.c_int, [c_void_p]),
    "mx_stream_sync": (ctypes.c_int, [c_void_p]),
    "mx_event_create": (ctypes.c_int, [P(c_void_p), c_int32]),
    "mx_event_record": (ctypes.c_int, [c_void_p, c_void_p]),
    "mx_event_wait": (ctypes.c_int, [c_void_p, c_void_p]),
    "mx_event_sync": (ctypes.c_int, [c_void_p]),
    "mx_event_query": (ctypes.c_int, [c_void_p, P(c_int32)]),
    "mx_event_destroy": (ctypes.c_int, [c_void_p]),
    "mx_event_elapsed_ms": (ctypes.c_int, [P(c_float), c_void_p, c_void_p]),
    "mx_moe_workspace_size": (ctypes.c_int, [P(MxMoeDesc), c_int32, P(c_size_t)]),
    "mx_moe_views": (ctypes.c_int, [P(MxMoeDesc), c_int32, c_void_p, P(MxMoeViews)]),
    "mx_moe_forward": (ctypes.c_int, [P(MxMoeDesc), P(MxMoeWeights), c_void_p, c_void_p,
                                      c_int32, c_void_p, c_size_t, c_void_p]),
    "mx_moe_forward_noalloc": (ctypes.c_int, [P(MxMoeDesc), P(MxMoeWeights), c_void_p,
                                              c_void_p, c_int32, c_void_p]),
    "mx_moe_forward_profiled": (ctypes.c_int, [P(MxMoeDesc), P(MxMoeWeights), c_void_p,
                                               c_void_p, c_int32, c_void_p, c_size_t,
                                               c_void_p, P(c_void_p), c_int32]),
    "mx_rmsnorm": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_float, c_int32, c_int32,
                                  c_void_p, c_void_p, c_void_p]),
    "mx_router_logits": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                        c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "mx_router_topk": (ctypes.c_int, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                      c_int32, c_int32, c_int32, c_float, c_int32, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "mx_dispatch": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                   c_int32, c_int32] + [c_void_p] * 12 + [c_void_p]),
    "mx_dispatch_scratch_size": (ctypes.c_int, [c_int32, c_int32, c_int32, P(c_size_t)]),
    "mx_dispatch_chunked": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                           c_int32, c_int32, c_int32, c_void_p] +
                            [c_void_p] * 12 + [c_void_p]),
    "mx_expert_gate_up": (ctypes.c_int, [P(MxMoeDesc), c_void_p, c_int32, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_int32, c_void_p, c_void_p]),
    "mx_expert_down": (ctypes.c_int, [P(MxMoeDesc), c_void_p, c_int32, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_int32, c_void_p, c_void_p]),
    "mx_combine": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                  c_int32, c_void_p, c_void_p]),
    "mx_fill_normal": (ctypes.c_int, [c_void_p, c_int32, c_size_t, c_uint64, c_uint64,
                                      c_uint64, c_float, c_void_p]),
    "mx_moe_forward_stages": (ctypes.c_int, [P(MxMoeDesc), P(MxMoeWeights), c_void_p, c_void_p,
                                             c_int32, c_void_p, c_size_t, c_int32, c_int32,
                                             c_void_p]),
    "mx_tile_weights": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "mx_quantize_rows_i8": (ctypes.c_int, [c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                           c_void_p, c_void_p]),
    "mx_linear_attn_workspace_size": (ctypes.c_int, [P(MxLinearAttnDesc), c_int32,
                                                     P(c_size_t)]),
    "mx_linear_attn_views": (ctypes.c_int, [P(MxLinearAttnDesc), c_int32, c_void_p,
                                            P(MxLinearAttnViews)]),
    "mx_linear_attn_forward": (ctypes.c_int, [P(MxLinearAttnDesc), P(MxLinearAttnWeights),
                                              c_void_p, c_void_p, c_int32, c_void_p, c_size_t,
                                              c_void_p]),
    "mx_linear_attn_forward_profiled": (ctypes.c_int, [P(MxLinearAttnDesc),
                                                       P(MxLinearAttnWeights), c_void_p,
                                                       c_void_p, c_int32, c_void_p, c_size_t,
                                                       c_void_p, P(c_void_p), c_int32]),
    "mx_full_attn_workspace_size": (ctypes.c_int, [P(MxFullAttnDesc), c_int32, P(c_size_t)]),
    "mx_full_attn_views": (ctypes.c_int, [P(MxFullAttnDesc), c_int32, c_void_p,
                                          P(MxFullAttnViews)]),
    "mx_full_attn_forward": (ctypes.c_int, [P(MxFullAttnDesc), P(MxFullAttnWeights), c_void_p,
                                            c_void_p, c_int32, c_void_p, c_size_t, c_void_p]),
    "mx_full_attn_forward_profiled": (ctypes.c_int, [P(MxFullAttnDesc), P(MxFullAttnWeights),
                                                     c_void_p, c_void_p, c_int32, c_void_p,
                                                     c_size_t, c_void_p, P(c_void_p), c_int32]),
    "mx_gated_delta_scan": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                           c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "mx_gated_delta_scan_workspace_size": (ctypes.c_int, [c_int32, c_int32, c_int32, c_int32,
                                                          P(c_size_t)]),
    "mx_gated_delta_scan_ws": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                              c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                              c_size_t, c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with every signature declared."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        lib_path = Path(path or os.environ.get("MX_LIB_PATH") or LIB_PATH)
        if not lib_path.exists():
            raise RuntimeError(
                f"{lib_path.name} is not built ({lib_path}); run __graft_entry__.build() "
                "or python -m moe_mi355x.build")
        lib = ctypes.CDLL(str(lib_path))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def error_string(status: int) -> str:
    return load().mx_error_string(int(status)).decode()


def check(status: int, what: str = "") -> None:
    """Raise for a non-zero library status (HIP errors -> RuntimeError)."""
    status = int(status)
    if status == MX_OK:
        return
    prefix = f"{what}: " if what else ""
    if status > 0:
        raise RuntimeError(f"{prefix}HIP runtime call failed with status={status} "
                           f"({error_string(status)})")
    if status in (MX_ERR_INVALID, MX_ERR_ALIGNMENT, MX_ERR_WORKSPACE):
        raise ValueError(f"{prefix}{error_string(status)} (status={status})")
    raise RuntimeError(f"{prefix}{error_string(status)} (status={status})")


def exported_names() -> list[str]:
    return list(_SIGNATURES)
