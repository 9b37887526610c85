"""Pinned host tensors through the library's hipHostMalloc.

Reference: specmoe/backend/pin_memory_allocator.py:7-65 -- the same functions, which there
load libcudart and support fp16/fp32 only. Here the allocation is smx_host_alloc
(hipHostMalloc, portable) on the HIP runtime PyTorch uses, and bfloat16 is supported (numpy has
no bfloat16: the buffer is wrapped as uint16 and viewed as torch.bfloat16).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _lib

_NP_OF = {torch.float16: np.float16, torch.float32: np.float32, torch.bfloat16: np.uint16}


def check_cuda_status(status: int) -> None:
    if status != 0:
        raise RuntimeError(f"HIP error: {status} ({_lib.lib().smx_error_string(status).decode()})")


def cuda_host_alloc(size_in_bytes: int) -> ctypes.c_void_p:
    """Pinned host memory of `size_in_bytes` bytes (free with free_pinned_tensor)."""
    ptr = ctypes.c_void_p()
    check_cuda_status(_lib.lib().smx_host_alloc(int(size_in_bytes), ctypes.byref(ptr)))
    return ptr


def make_pinned_numpy_array(ptr: ctypes.c_void_p, size: int, dtype=np.float32) -> np.ndarray:
    """A numpy view of `size` elements of `dtype` at `ptr` (no copy, no ownership)."""
    buffer_type = ctypes.c_char * (size * np.dtype(dtype).itemsize)
    buffer = buffer_type.from_address(ptr.value)
    return np.frombuffer(buffer, dtype=dtype, count=size)


def make_pinned_tensor(size_in_bytes=2.625 * 1024 * 1024 * 1024, dtype=torch.float16):
    """(tensor, ptr): a 1-D CPU tensor of `dtype` over freshly pinned memory; the caller frees
    `ptr` with free_pinned_tensor once the tensor is no longer used."""
    if dtype not in _NP_OF:
        raise ValueError(f"Unsupported dtype: {dtype}")
    element_size = torch.tensor([], dtype=dtype).element_size()
    total_bytes = int(size_in_bytes)
    num_elements = total_bytes // element_size
    ptr = cuda_host_alloc(total_bytes)
    arr = make_pinned_numpy_array(ptr, num_elements, dtype=_NP_OF[dtype])
    tensor = torch.from_numpy(arr)
    if dtype == torch.bfloat16:
        tensor = tensor.view(torch.bfloat16)
    return tensor, ptr


def free_pinned_tensor(ptr: ctypes.c_void_p) -> None:
    check_cuda_status(_lib.lib().smx_host_free(ptr))
