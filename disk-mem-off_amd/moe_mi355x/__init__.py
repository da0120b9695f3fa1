"""MI355X (gfx950) MoE-layer hot path behind the offload-runtime executor API.

Compute runs only in ``libmoe_mi355x.so`` (HIP kernels, C ABI, see include/moe_mi355x.h);
this package is the host side: backend, pools, runtime, layer layout and executors.
"""
from .activations import DeviceActivations
from .backends import DeviceBackend, MI355XBackend, ROCmBackend, detect_backend
from .buffer_pool import DeviceBufferPool
from .pinned_pool import PinnedHostBufferPool
from .executors import (GLM4MoeExecutor, Qwen3NextExecutor, host_attention, host_dense,
                        read_layer_tensors)
from .layout import MoeLayerLayout, make_layer_spec, pack_tensors, unpack_host
from .moe import ROUTER_MODES, MoeConfig, MoeRunner
from .quantize import (CompositeDequantizer, Float16Dequantizer, Int8Dequantizer,
                       dequantize_rows_int8, quantize_moe_tensors, quantize_rows_int8)
from .runtime import LayerExecutor, LayerMetrics, OffloadRuntime, RuntimeMetrics
from .scheduler import LookaheadScheduler, PrefetchScheduler
from .storage import DeviceResidentStorage, InMemoryStorage, LayerStorage
from .types import DeviceBuffer, HostBuffer, LayerSpec

__all__ = [
    "CompositeDequantizer", "DeviceActivations", "DeviceBackend", "DeviceBuffer",
    "DeviceBufferPool", "DeviceResidentStorage",
    "Float16Dequantizer", "GLM4MoeExecutor", "HostBuffer", "InMemoryStorage", "Int8Dequantizer",
    "LayerExecutor", "LayerMetrics", "LayerSpec", "LayerStorage", "LookaheadScheduler",
    "MI355XBackend", "MoeConfig", "MoeLayerLayout", "MoeRunner",
    "OffloadRuntime", "PinnedHostBufferPool", "PrefetchScheduler", "Qwen3NextExecutor",
    "ROCmBackend", "ROUTER_MODES", "RuntimeMetrics", "dequantize_rows_int8", "detect_backend",
    "host_attention", "host_dense", "make_layer_spec", "pack_tensors", "quantize_moe_tensors",
    "quantize_rows_int8", "read_layer_tensors", "unpack_host",
]
