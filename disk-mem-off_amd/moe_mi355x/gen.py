"""Portable counter-based normal generator for synthetic inputs and weights.

Element ``i`` of stream ``(seed, stream_id)`` depends only on those three integers, so
any slice can be produced independently and the device twin ``mx_fill_normal``
(csrc/mx_synth.hip) produces the same numbers:

    key = mix(mix(seed) ^ (stream_id * 0xD1B54A32D192ED03))
    x0  = mix(key + 2c * G),  x1 = mix(key + (2c + 1) * G),   c = offset + i
    u1  = ((x0 >> 11) + 1) * 2**-53  in (0, 1],   u2 = (x1 >> 11) * 2**-53  in [0, 1)
    z   = sqrt(-2 ln u1) * cos(2 pi u2)             (Box-Muller, float64)
    out = float32(std * z)   [float16(out) for fp16]

``mix`` is the SplitMix64 finaliser, ``G = 0x9E3779B97F4A7C15`` and ``std`` is taken as
a float32 value.  All integer arithmetic is modulo 2**64.
"""
from __future__ import annotations

import numpy as np

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_K = np.uint64(0xD1B54A32D192ED03)
_S30, _S27, _S31, _S11 = (np.uint64(s) for s in (30, 27, 31, 11))
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> _S30)) * _M1
    z = (z ^ (z >> _S27)) * _M2
    return z ^ (z >> _S31)


def stream_key(seed: int, stream_id: int) -> int:
    with np.errstate(over="ignore"):
        s = _mix(np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))
        k = _mix(s ^ (np.array([stream_id & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64) * _K))
    return int(k[0])


def normal(seed: int, stream_id: int, shape, std: float = 1.0, offset: int = 0,
           dtype=np.float32) -> np.ndarray:
    """Normals of stream (seed, stream_id) starting at element ``offset``."""
    n = int(np.prod(shape, dtype=np.int64))
    key = np.uint64(stream_key(seed, stream_id))
    std64 = float(np.float32(std))
    out = np.empty(n, dtype=np.float32)
    with np.errstate(over="ignore"):
        for b in range(0, n, _CHUNK):
            e = min(n, b + _CHUNK)
            c = np.arange(offset + b, offset + e, dtype=np.uint64)
            x0 = _mix(key + (np.uint64(2) * c) * _G)
            x1 = _mix(key + (np.uint64(2) * c + np.uint64(1)) * _G)
            u1 = ((x0 >> _S11) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
            u2 = (x1 >> _S11).astype(np.float64) * 2.0 ** -53
            z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
            out[b:e] = (std64 * z).astype(np.float32)
    out = out.reshape(shape)
    if np.dtype(dtype) == np.float16:
        return out.astype(np.float16)
    if np.dtype(dtype) != np.float32:
        return out.astype(dtype)
    return out
