"""Shared test setup: import paths, the ``gpu`` marker, common fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "disk-mem-off_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmoe_mi355x.so)")


@pytest.fixture(scope="session")
def mi355x():
    """The ROCm backend on device 0 (GPU tests only; fails loudly without the library)."""
    from moe_mi355x.backends import MI355XBackend

    return MI355XBackend(0)


@pytest.fixture(scope="session")
def stream(mi355x):
    s = mi355x.create_stream("test")
    yield s
    mi355x.synchronize_stream(s)
    mi355x.destroy_stream(s)
