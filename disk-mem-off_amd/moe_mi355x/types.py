"""Layer and buffer descriptors shared by the runtime, backends and executors.

Same fields and meaning as offload_runtime/types.py:7-29 (``LayerSpec``, ``HostBuffer``,
``DeviceBuffer``) so layer lists and buffers move between the two packages unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any


@dataclass(frozen=True)
class LayerSpec:
    """One offloadable layer: id, name, byte size of its packed weights, metadata.

    ``metadata["tensors"]`` lists ``{name, shape, dtype, offset, nbytes}`` entries that
    locate each tensor inside the packed layer buffer (loader/huggingface.py:498-506).
    """

    layer_id: int
    name: str
    nbytes: int
    metadata: dict[str, Any] = field(default_factory=dict)


@dataclass
class HostBuffer:
    """Host bytes (``memoryview``); ``pinned`` marks page-locked memory."""

    view: memoryview
    pinned: bool = False

    @property
    def nbytes(self) -> int:
        return self.view.nbytes


@dataclass
class DeviceBuffer:
    """Device allocation: ``handle`` is the integer device address on this backend."""

    handle: Any
    nbytes: int
    backend: str
