"""The C-ABI library loads and exports every entry point include/moe_mi355x.h declares;
host-side argument validation (no GPU work) behaves as documented."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from moe_mi355x import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "moe_mi355x.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "mx_moe_forward" in names and "mx_malloc" in names and len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"symbols declared but not exported: {missing}"


def test_bindings_cover_the_header():
    assert set(declared_functions()) == set(_lib.exported_names())


def _desc(**kw):
    d = dict(hidden=64, inter=32, shared_inter=32, n_experts=8, top_k=2, router_mode=0,
             norm_topk_prob=1, weight_dtype=_lib.MX_DT_F16, param_dtype=_lib.MX_DT_F32,
             has_bias=1, has_shared_gate=0, routed_scaling=2.5, eps=1e-5)
    d.update(kw)
    return _lib.MxMoeDesc(**d)


def _ws(desc, T):
    n = ctypes.c_size_t()
    rc = _lib.load().mx_moe_workspace_size(ctypes.byref(desc), T, ctypes.byref(n))
    return rc, n.value


def test_workspace_size_grows_with_tokens():
    d = _desc()
    rc1, n1 = _ws(d, 1)
    rc2, n2 = _ws(d, 4096)
    assert rc1 == rc2 == _lib.MX_OK and 0 < n1 < n2


@pytest.mark.parametrize("field,value", [("top_k", 0), ("top_k", 9), ("router_mode", 3),
                                         ("weight_dtype", 7), ("param_dtype", 2),
                                         ("hidden", 0), ("n_experts", -1)])
def test_bad_descriptor_is_rejected(field, value):
    rc, _ = _ws(_desc(**{field: value}), 8)
    assert rc == _lib.MX_ERR_INVALID


def test_shared_gate_needs_shared_expert():
    rc, _ = _ws(_desc(shared_inter=0, has_shared_gate=1), 8)
    assert rc == _lib.MX_ERR_INVALID


def test_null_pointers_rejected_before_any_launch():
    lib = _lib.load()
    assert lib.mx_rmsnorm(None, None, 0, 1e-5, 4, 64, None, None, None) == _lib.MX_ERR_INVALID
    assert lib.mx_combine(None, None, None, 4, 64, 2, 0, None, None) == _lib.MX_ERR_INVALID
    assert lib.mx_malloc(None, 16) == _lib.MX_ERR_INVALID
    d = _desc()
    w = _lib.MxMoeWeights()
    assert lib.mx_moe_forward(ctypes.byref(d), ctypes.byref(w), None, None, 4, None, 0,
                              None) == _lib.MX_ERR_INVALID


def test_error_strings():
    assert _lib.error_string(_lib.MX_ERR_WORKSPACE) == "workspace too small"
    with pytest.raises(ValueError):
        _lib.check(_lib.MX_ERR_INVALID, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.MX_ERR_UNSUPPORTED, "x")


def test_noalloc_refuses_batches_beyond_its_scratch_on_the_host():
    """mx_moe_forward_noalloc checks the batch's workspace against its fixed scratch before
    any HIP call: an oversized batch or a bad descriptor is refused here, without a GPU."""
    lib = _lib.load()
    w = _lib.MxMoeWeights()
    big = _desc(hidden=5120, inter=1536, shared_inter=1536, n_experts=160, top_k=8)
    T = 1
    while _ws(big, T)[1] <= _lib.MX_NOALLOC_MAX_WORKSPACE:
        T *= 2
    assert lib.mx_moe_forward_noalloc(ctypes.byref(big), ctypes.byref(w), None, None, T,
                                      None) == _lib.MX_ERR_WORKSPACE
    assert lib.mx_moe_forward_noalloc(ctypes.byref(_desc(top_k=0)), ctypes.byref(w), None,
                                      None, 4, None) == _lib.MX_ERR_INVALID
