"""Shared helpers for the GPU parity tests: torch <-> oracle conversions and input builders."""
from __future__ import annotations

import json
import os

import numpy as np
import torch

from oracle import moe_ref as ref

TORCH_TO_ORACLE = {torch.bfloat16: ref.BF16, torch.float16: ref.F16, torch.float32: ref.F32}


def to_oracle(t: torch.Tensor) -> np.ndarray:
    """GPU/CPU tensor -> numpy array the oracle reads (uint16 bits for 16-bit types)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def f32_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def max_rel_err(y: np.ndarray, want: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the parity metric of the layer outputs)."""
    denom = float(np.abs(want).max())
    return float(np.abs(y.astype(np.float64) - want.astype(np.float64)).max()) / max(denom, 1e-30)


# Output tolerance per activation dtype: max |y - ref| / max |ref|. bf16 carries 8 mantissa
# bits and four rounding points; the layer's bf16 parity bound is 1e-2.
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-4}
TOL_BY_NAME = {"bf16": 1e-2, "f16": 2e-3, "f32": 1e-4}


def elem_rel_err(y: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Elementwise |y - ref| / max(|ref|, 1e-3 * max|ref|): the relative error of every output,
    with a floor so that outputs near zero are measured against the output scale."""
    want = want.astype(np.float64)
    floor = 1e-3 * max(float(np.abs(want).max()), 1e-30)
    return np.abs(y.astype(np.float64) - want) / np.maximum(np.abs(want), floor)


# The 99th percentile of the elementwise relative error may reach this multiple of the
# output tolerance: outputs near the floor of elem_rel_err carry a larger relative rounding
# error than the largest ones, but 99 in 100 outputs stay within a small multiple of it.
P99_FACTOR = 2.0


def parity(y: np.ndarray, want: np.ndarray, tol: float, case: str = "", elementwise: bool = True,
           **extra) -> dict:
    """Both output metrics of one comparison. Asserts max |y - ref| / max |ref| <= tol and
    (with `elementwise`) the 99th percentile of the elementwise relative error <= P99_FACTOR *
    tol, and records the figures: with SMX_PARITY_LOG set, one JSON line per comparison is
    appended to that file. `elementwise=False` is for outputs of a chain of layers compared
    end to end: the inputs of its later layers already differ, and the propagated absolute
    error makes the relative error of small outputs large by construction (each layer is
    compared elementwise on its own input)."""
    el = elem_rel_err(y, want)
    rec = {"case": case, "max_rel_err": max_rel_err(y, want), "tol": tol,
           "elem_rel_err_median": float(np.median(el)), "elem_rel_err_p99": float(np.quantile(el, 0.99)),
           "elem_rel_err_max": float(el.max()), "outputs": int(el.size), **extra}
    path = os.environ.get("SMX_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert rec["max_rel_err"] <= tol, rec
    if elementwise:
        assert rec["elem_rel_err_p99"] <= P99_FACTOR * tol, rec
    return rec


def nan_buffers(x: torch.Tensor, nbytes: int):
    """An output like x filled with NaN and a workspace of nbytes bytes of 0xFF (a NaN in
    every float type), so that a kernel that reads a row the call did not write gives NaN."""
    out = torch.full_like(x, float("nan"))
    ws = torch.full((max(int(nbytes), 1),), 0xFF, dtype=torch.uint8, device=x.device)
    return out, ws


def make_pool(E: int, H: int, I: int, dtype: torch.dtype, num_slots: int | None = None,
              seed: int = 0, scale: float = 0.02, device: str = "cuda"):
    """Pool [P, 3*I*H] of N(0, scale) pages and a permuted expert->slot map (int64)."""
    P = num_slots or E
    g = torch.Generator(device=device).manual_seed(seed)
    pool = (torch.randn((P, 3 * I * H), generator=g, device=device, dtype=torch.float32) * scale).to(dtype)
    gc = torch.Generator().manual_seed(seed + 1)
    slots = torch.randperm(P, generator=gc)[:E].to(device=device, dtype=torch.int64)
    return pool, slots


def zipf_gate_logits(x: torch.Tensor, E: int, s: float = 1.2, seed: int = 0) -> torch.Tensor:
    """Router logits x Wg^T + b, Wg ~ N(0, 0.02), b_e = ln p_e with p_e ~ (e+1)^-s (a skewed
    expert load), computed in x's dtype."""
    g = torch.Generator(device=x.device).manual_seed(seed + 7)
    wg = (torch.randn((E, x.shape[1]), generator=g, device=x.device) * 0.02).to(x.dtype)
    p = torch.arange(1, E + 1, dtype=torch.float64) ** (-s)
    b = torch.log(p / p.sum()).to(device=x.device, dtype=x.dtype)
    return torch.nn.functional.linear(x, wg) + b
