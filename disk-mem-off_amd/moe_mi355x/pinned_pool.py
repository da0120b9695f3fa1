"""Pinned host buffer pool (module path of offload_runtime/pinned_pool.py)."""
from .buffer_pool import PinnedHostBufferPool

__all__ = ["PinnedHostBufferPool"]
