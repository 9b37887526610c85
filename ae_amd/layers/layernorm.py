"""RMSNorm with the reference's interface, computed by the library's norm kernel.

Reference: specmoe/layers/layernorm.py:7-52. ``forward(x, residual=None)``: with a residual,
``residual = x + residual`` and ``x = rmsnorm(residual)`` are written in place and
``(x, residual)`` is returned (sglang's fused_add_rmsnorm, :31); without one, a new
normalized tensor is returned. The arithmetic is the reference's forward_native (:36-52):
fp32 sum, mean of squares, ``x * rsqrt(var + eps) * weight`` rounded once.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
from torch import nn

from .. import _lib
from ._torch import dtype_code, ptr, require_gpu, stream_of


def add_rmsnorm_gate(hidden: torch.Tensor, residual: Optional[torch.Tensor],
                     norm_weight: torch.Tensor, eps: float,
                     gate_weight: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Residual add + RMSNorm (+ router gate) in one kernel. Writes the normalized states to
    ``out`` (default: ``hidden``, in place) and the sum to ``residual``; returns the router
    logits ``[T, E]`` when ``gate_weight`` ``[E, H]`` is given."""
    assert hidden.dim() == 2 and hidden.is_contiguous(), "hidden states must be [T, H] contiguous"
    T, H = hidden.shape
    require_gpu(hidden, residual, norm_weight, gate_weight, out)
    for t in (residual, norm_weight, gate_weight, out):
        if t is not None:
            assert t.dtype == hidden.dtype and t.is_contiguous(), "dtype/contiguity mismatch"
    assert norm_weight.numel() == H
    if residual is not None:
        assert residual.shape == hidden.shape
    out = hidden if out is None else out
    logits = None
    E = 0
    if gate_weight is not None:
        E = gate_weight.shape[0]
        assert gate_weight.shape == (E, H)
        logits = torch.empty((T, E), dtype=hidden.dtype, device=hidden.device)
    _lib.call("smx_add_rmsnorm_gate", ptr(hidden), ptr(residual), ptr(out), dtype_code(hidden.dtype),
              T, H, ptr(norm_weight), float(eps), ptr(gate_weight), E, ptr(logits), stream_of(hidden))
    return logits


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        if x.device.type == "cuda":
            return self.forward_cuda(x, residual)
        return self.forward_native(x, residual)

    def forward_cuda(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None
                     ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        shape = x.shape
        x2 = x.view(-1, shape[-1])
        w = self.weight.data
        if w.dtype != x.dtype:
            w = w.to(x.dtype)
        if residual is not None:
            add_rmsnorm_gate(x2, residual.view(-1, shape[-1]), w, self.variance_epsilon)
            return x, residual
        out = torch.empty_like(x2)
        add_rmsnorm_gate(x2, None, w, self.variance_epsilon, out=out)
        return out.view(shape)

    def forward_native(self, *args, **kwargs):
        raise NotImplementedError("this build has no CPU RMSNorm path")
