"""Compile the HIP sources of the MoE hot path into ``libmoe_mi355x.so`` (gfx950).

Each ``csrc/*.hip`` file is compiled to an object with ``hipcc --offload-arch=gfx950`` in
parallel, then linked into a shared library next to this file.  Run as a module
(``python -m moe_mi355x.build``) or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_ROOT = PKG_DIR.parent  # disk-mem-off_amd/
CSRC = SRC_ROOT / "csrc"
INCLUDE = SRC_ROOT.parent / "include"
LIB_NAME = "libmoe_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = SRC_ROOT / "_build"
ARCH = os.environ.get("MX_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: packed fp32 VALU forms are kept out of every kernel.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


# No vendor libraries: every kernel is this package's own.
LINK_LIBS: list[str] = []


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, hipcc: str) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link ``libmoe_mi355x.so``; return its path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), *LINK_LIBS,
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
