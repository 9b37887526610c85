"""Build, load and call the C++ CPU restatement of the MoE layer (oracle/cpu_moe.cpp) -- a timed
CPU baseline. MEASUREMENT AND TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only bench.py's cpu_baseline leg (as the thing timed on the host cores) and tests/ (which pin it
against the numpy oracle in moe_ref.py) may import this module. The product path (ae_amd) never
imports it and has no CPU fallback.

cpu_moe.cpp writes the layer as the reference writes its one CPU kernel
(specmoe/csrc/flashattention.cpp:163-207): cblas_sgemm for each contraction, OpenMP over the
independent work. Its MKL is the image's libmkl_rt (/opt/conda/lib; mkl.h is not installed, so
the CBLAS prototype is declared in the source): loaded here with RTLD_GLOBAL before the library,
on MKL's sequential layer, so the library's OpenMP threads are the only ones. Built with g++ into
oracle/libcpu_moe.so (build(); __graft_entry__.build() calls it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpu_moe.cpp")
LIB = os.path.join(HERE, "libcpu_moe.so")
MKL = "/opt/conda/lib/libmkl_rt.so.1"

_lib: Optional[ctypes.CDLL] = None


def available() -> bool:
    return os.path.exists(MKL)


def build() -> str:
    """g++ -> oracle/libcpu_moe.so (no MKL at link time: cblas_sgemm binds at load)."""
    cmd = ["g++", "-O3", "-mavx2", "-mfma", "-fopenmp", "-shared", "-fPIC", "-std=c++17", "-Wall",
           SRC, "-o", LIB + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{proc.stderr}")
    os.replace(LIB + ".tmp", LIB)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not available():
            raise RuntimeError(f"{MKL} not found")
        if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
            build()
        os.environ["MKL_THREADING_LAYER"] = "SEQUENTIAL"
        ctypes.CDLL(MKL, mode=ctypes.RTLD_GLOBAL)
        h = ctypes.CDLL(LIB)
        fp = ctypes.c_void_p
        h.cpu_moe_forward.restype = ctypes.c_int
        h.cpu_moe_forward.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, fp, ctypes.c_int, fp, fp, fp, ctypes.c_int,
                                      ctypes.c_int, fp, fp, fp]
        _lib = h
    return _lib


class MklCpuMoE:
    """One MoE layer (no shared expert) on the host through cpu_moe.cpp. `w1`, `w3`, `w2`: per
    expert fp32 matrices ([I, H], [I, H], [H, I], C-contiguous numpy or torch CPU tensors), or
    missing for an expert without a pool page."""

    def __init__(self, w1: dict, w3: dict, w2: dict, E: int, H: int, I: int, dtype: str,
                 threads: int = 0):
        if dtype not in ("bf16", "f32"):
            raise ValueError("the C++ restatement rounds to bf16 or not at all")
        self.E, self.H, self.I, self.bf16, self.threads = E, H, I, int(dtype == "bf16"), threads
        self._keep = []

        def ptrs(ws):
            arr = (ctypes.c_void_p * E)()
            for e in range(E):
                if e in ws:
                    a = ws[e]
                    a = a.numpy() if hasattr(a, "numpy") else a
                    assert a.dtype == np.float32 and a.flags.c_contiguous
                    self._keep.append(a)
                    arr[e] = a.ctypes.data
            return arr
        self.p1, self.p3, self.p2 = ptrs(w1), ptrs(w3), ptrs(w2)

    def forward(self, x: np.ndarray, logits: np.ndarray, top_k: int, renormalize: bool):
        """x [T, H] fp32 (bf16 values for a bf16 layer), logits [T, E] fp32 -> (y, w, ids)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        T = x.shape[0]
        y = np.empty((T, self.H), np.float32)
        w = np.empty((T, top_k), np.float32)
        ids = np.empty((T, top_k), np.int32)
        rc = lib().cpu_moe_forward(x.ctypes.data, T, self.H, self.I, self.E, top_k, logits.ctypes.data,
                                   int(bool(renormalize)), self.p1, self.p3, self.p2, self.bf16,
                                   self.threads, y.ctypes.data, w.ctypes.data, ids.ctypes.data)
        if rc != 0:
            raise ValueError(f"cpu_moe_forward returned {rc}")
        return y, w, ids
