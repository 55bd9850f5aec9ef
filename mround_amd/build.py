"""Builds ``libmround_hip.so`` for gfx950 from ``mround_amd/csrc/*.hip`` (device
kernels, compiled by ``hipcc``) and ``mround_amd/csrc/*.cpp`` (host-only code,
compiled by ``g++``).

Each source is compiled into an object in ``mround_amd/_build``
(in parallel), then linked into ``mround_amd/_lib/libmround_hip.so``, in tree,
so that the library travels with the source tree. Run as
``python -m mround_amd.build`` or through ``__graft_entry__.build()``.

Flags that matter for correctness:

* ``-ffp-contract=off`` -- the quantizer's arithmetic must round operation by
  operation as the reference's float32 arithmetic does; a contracted
  multiply-add would change codes.
* ``-fhip-fp32-correctly-rounded-divide-sqrt`` -- IEEE division (the HIP
  default, stated explicitly).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` -- no packed fp32 ALU
  instructions are generated.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ_DIR = PKG / "_build"
LIB_DIR = PKG / "_lib"
LIB_PATH = LIB_DIR / "libmround_hip.so"
ARCH = os.environ.get("MROUND_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    if src.suffix == ".cpp":
        cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
        cmd = [cxx, *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
