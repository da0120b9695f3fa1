"""Layer storage (protocol of offload_runtime/storage/base.py:8-21) and the in-memory
store used by tests and the streaming bench (offload_runtime/storage/in_memory.py:6-26)."""
from __future__ import annotations

from typing import Any, Protocol

from .types import HostBuffer


class LayerStorage(Protocol):
    def request(self, layer_id: int) -> None: ...

    def wait(self, layer_id: int) -> None: ...

    def get(self, layer_id: int) -> HostBuffer: ...

    def release(self, layer_id: int) -> None: ...


class InMemoryStorage:
    """Serves layer bytes from memory.  Values may be ``bytes`` / ``bytearray`` or
    ready ``HostBuffer`` objects (for example pinned buffers)."""

    def __init__(self, layer_bytes: dict[int, Any]) -> None:
        self._layer_bytes = layer_bytes

    def request(self, layer_id: int) -> None:
        return None

    def wait(self, layer_id: int) -> None:
        return None

    def get(self, layer_id: int) -> HostBuffer:
        payload = self._layer_bytes[layer_id]
        if isinstance(payload, HostBuffer):
            return payload
        return HostBuffer(view=memoryview(payload), pinned=False)

    def release(self, layer_id: int) -> None:
        return None

    def get_disk_read_ms(self, layer_id: int) -> float:
        return 0.0


class DeviceResidentStorage:
    """Layers kept resident in device memory (a model whose layers fit in HBM, or the hot
    subset of one): ``get`` returns the layer's ``DeviceBuffer``, which the runtime hands to
    the executor without a copy and never frees or re-pools (the store keeps it).  Same
    ``LayerStorage`` protocol; no counterpart in the reference, whose runtime copies every
    layer from host storage."""

    def __init__(self, buffers: dict[int, Any]) -> None:
        self._buffers = buffers

    def request(self, layer_id: int) -> None:
        return None

    def wait(self, layer_id: int) -> None:
        return None

    def get(self, layer_id: int) -> Any:
        return self._buffers[layer_id]

    def release(self, layer_id: int) -> None:
        return None

    def get_disk_read_ms(self, layer_id: int) -> float:
        return 0.0
