"""Torch plumbing for the C ABI: dtype codes, raw pointers, the current HIP stream."""
from __future__ import annotations

import ctypes

import torch

from .. import _lib

_DTYPE_CODE = {
    torch.float32: _lib.SMX_F32,
    torch.float16: _lib.SMX_F16,
    torch.bfloat16: _lib.SMX_BF16,
}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    """The current torch stream of t's device, as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Per-call scratch from torch's caching allocator (reused across calls, no hipMalloc)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
