"""Build recipe for libspecmoe_mi355x.so (gfx950) -- compiles in-tree, no JIT cache.

    python -m ae_amd.build          # or: from ae_amd.build import build_library
    python -m ae_amd.build --changed   # recompile only sources newer than their objects

Each HIP source is compiled to an object under ae_amd/_build/ (in parallel), then linked
into ae_amd/libspecmoe_mi355x.so. hipcc cross-compiles, so this runs without a GPU.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libspecmoe_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["routing.hip", "experts.hip", "layer1.hip", "tiles.hip", "capi.hip", "transfer.hip",
           "stream_probe.hip"]
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every HIP translation unit (the host pass warns
# that it does not know the feature; that warning is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build the library")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def _stale(src: str) -> bool:
    """The object of src is missing or older than src or any header in csrc/ or include/."""
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    if not os.path.exists(obj):
        return True
    deps = [os.path.join(CSRC, src)]
    deps += [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    inc = os.path.join(os.path.dirname(PKG_DIR), "include")
    deps += [os.path.join(inc, h) for h in os.listdir(inc) if h.endswith(".h")]
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps)


def build_library(verbose: bool = False, changed_only: bool = False) -> str:
    """Compile the sources (all of them, or with changed_only those whose objects are stale)
    and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    todo = [s for s in SOURCES if _stale(s)] if changed_only else list(SOURCES)
    if todo:
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(todo)) as ex:
            list(ex.map(_compile, todo))
    if verbose and changed_only:
        print(f"compiled {todo}")
    objs = [os.path.join(BUILD_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)  # atomic: a concurrent loader never sees a half-written file
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True, changed_only="--changed" in sys.argv[1:])
    sys.exit(0)
