"""Activations that stay on the device between consecutive layers.

The reference hands NumPy ``[T, H]`` fp32 arrays from layer to layer
(offload_runtime/runtime.py:169-175, glm4_moe.py:244-245), so a device executor pays one
upload and one read-back per layer.  A ``DeviceActivations`` is what an executor built
with ``device_activations=True`` returns instead: fp32 ``[T, H]`` rows at a device address
owned by the executor.  Passed to the next layer's ``run_layer`` it is read in place;
``numpy()`` (or ``np.asarray``) synchronises the stream that wrote it and copies it back.

A handle is valid until the buffer behind it is written again: the executor alternates
between two output buffers, so the output of layer i stays readable while layer i + 1
runs and is overwritten by layer i + 2.  A stale handle raises ``RuntimeError``.
"""
from __future__ import annotations

from typing import Any

import numpy as np


class DeviceActivations:
    """fp32 ``[tokens, hidden]`` activations resident on the device."""

    def __init__(self, owner: Any, slot: int, generation: int, ptr: int, tokens: int,
                 hidden: int, stream: Any) -> None:
        self._owner = owner
        self._slot = slot
        self._generation = generation
        self.ptr = int(ptr)
        self.shape = (int(tokens), int(hidden))
        self.stream = stream
        self.dtype = np.dtype(np.float32)

    @property
    def nbytes(self) -> int:
        return self.shape[0] * self.shape[1] * 4

    @property
    def valid(self) -> bool:
        return self._owner.generation(self._slot) == self._generation

    def check(self) -> None:
        if not self.valid:
            raise RuntimeError("DeviceActivations: the device buffer was overwritten by a "
                               "later layer (a handle is valid for one following layer)")

    def numpy(self) -> np.ndarray:
        """Copy to the host (synchronises the stream that produced the activations)."""
        self.check()
        out = np.empty(self.shape, np.float32)
        if out.size:
            backend = self._owner.backend
            backend.copy_d2h_ptr_async(out.ctypes.data, self.ptr, out.nbytes, self.stream)
            backend.synchronize_stream(self.stream)
        self.check()
        return out

    def __array__(self, dtype: Any = None, copy: Any = None) -> np.ndarray:
        out = self.numpy()
        return out if dtype is None else out.astype(dtype, copy=False)

    def __len__(self) -> int:
        return self.shape[0]

    def __repr__(self) -> str:
        return (f"DeviceActivations(shape={self.shape}, ptr={self.ptr:#x}, "
                f"valid={self.valid})")
