"""Counter-based generator: determinism, independent slices, moments, pinned values."""
from __future__ import annotations

import numpy as np

from moe_mi355x import gen


def test_deterministic_and_sliceable():
    a = gen.normal(7, 3, (64, 100))
    b = gen.normal(7, 3, (64, 100))
    assert np.array_equal(a, b)
    part = gen.normal(7, 3, (300,), offset=1000)
    assert np.array_equal(a.ravel()[1000:1300], part)


def test_streams_differ_and_moments():
    a = gen.normal(1, 1, (200000,))
    b = gen.normal(1, 2, (200000,))
    assert not np.array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert abs(np.corrcoef(a, b)[0, 1]) < 0.01
    s = gen.normal(1, 1, (200000,), std=0.02)
    np.testing.assert_allclose(s, (0.02 * a.astype(np.float64)).astype(np.float32), rtol=1e-6)


def test_fp16_is_rounded_fp32():
    a = gen.normal(5, 9, (1000,), std=0.02)
    h = gen.normal(5, 9, (1000,), std=0.02, dtype=np.float16)
    assert np.array_equal(h, a.astype(np.float16))


def test_first_values_are_pinned():
    # SplitMix64 -> Box-Muller values of stream (seed 0, stream 0); a change of the
    # generator would silently change every synthetic workload and golden input.
    v = gen.normal(0, 0, (4,))
    key = gen.stream_key(0, 0)
    mask = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)

    G = 0x9E3779B97F4A7C15
    for c in range(4):
        x0 = mix((key + 2 * c * G) & mask)
        x1 = mix((key + (2 * c + 1) * G) & mask)
        u1 = ((x0 >> 11) + 1) * 2.0 ** -53
        u2 = (x1 >> 11) * 2.0 ** -53
        z = np.sqrt(-2 * np.log(u1)) * np.cos(2 * np.pi * u2)
        assert v[c] == np.float32(z)
    assert key == mix(mix(0) ^ 0)
