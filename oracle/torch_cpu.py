"""Torch-CPU restatement of the MoE layer -- the timed CPU baseline. MEASUREMENT AND TEST
INFRASTRUCTURE, NOT PRODUCT CODE.

Only bench.py's cpu_baseline leg (as the thing timed on the host cores) and tests/ (which pin
it against the numpy oracle in moe_ref.py) may import this module. The product path (ae_amd)
never imports it and has no CPU fallback.

The reference has no CPU expert path: its FusedMoE.forward_cpu is unreachable
(specmoe/layers/FusedMoE.py:210-240) and specmoe/csrc holds only CPU attention. This module is
the same arithmetic as the oracle, written the way a CPU implementation of
stack_fused_moe (specmoe/layers/fused_moe_kernel.py:253-349) would be: torch tensor ops whose
GEMMs run on MKL, expert weights unpacked from the pool pages to fp32 once at construction
(outside any timed region), then per call

  routing   fp32 softmax over the experts, top-k by a stable descending sort (ties to the lower
            expert index), optional w / sum(w)  (select_experts, FusedMoE.py:174-185);
  experts   per active expert e and its assignments f = t*k + j in ascending order:
            g = round(x_t W1_e^T), u = round(x_t W3_e^T)             (:332-335, :203)
            a = round(silu(g) * u)                                  (:337)
            c3[t, j] = round((a W2_e^T) * w[t, j])                   (:339-342, :197-201)
  combine   y = round(sum_j c3[:, j])  (fp32, j in order)            (:344-347)

round() is to the activation dtype (bf16 / fp16; fp32 rounds nowhere). The shared-expert blocks
(Qwen1.5-MoE, DeepSeek-V2; no reference code) follow the oracle's rounding points:
y = round(round(routed * scale) + round(s * d)) with d the shared SwiGLU MLP and s the rounded
sigmoid of the shared gate logit (or 1).
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

_TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _round(t: torch.Tensor, dtype: str) -> torch.Tensor:
    """Round an fp32 tensor to `dtype` (nearest even) and back to fp32."""
    if dtype == "f32":
        return t
    return t.to(_TORCH[dtype]).to(torch.float32)


def _to_f32(a, dtype: str) -> torch.Tensor:
    """numpy (uint16 bit patterns for 16-bit types, or floats) or torch -> fp32 CPU tensor."""
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu", torch.float32)
    a = np.asarray(a)
    if dtype in ("bf16", "f16") and a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(_TORCH[dtype]).to(torch.float32)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def _silu(g: torch.Tensor) -> torch.Tensor:
    return g / (1.0 + torch.exp(-g))


class TorchCpuMoE:
    """One MoE layer on the host: the pool's pages as fp32 (W1, W3, W2) per expert."""

    def __init__(self, pool, slots, H: int, dtype: str, shared_page=None):
        self.dtype = dtype
        self.H = H
        slots = np.asarray(slots).reshape(-1)
        pool_f = pool if isinstance(pool, torch.Tensor) else None
        self.w1, self.w3, self.w2 = {}, {}, {}
        for e, slot in enumerate(slots):
            slot = int(slot)
            if not 0 <= slot < (pool_f.shape[0] if pool_f is not None else np.asarray(pool).shape[0]):
                continue
            page = _to_f32(pool_f[slot] if pool_f is not None else np.asarray(pool)[slot], dtype)
            I = page.numel() // (3 * H)
            self.w1[e] = page[: I * H].view(I, H).contiguous()
            self.w3[e] = page[I * H: 2 * I * H].view(I, H).contiguous()
            self.w2[e] = page[2 * I * H:].view(H, I).contiguous()
        self.E = slots.size
        self.shared = None
        if shared_page is not None:
            page = _to_f32(shared_page, dtype)
            Is = page.numel() // (3 * H)
            self.shared = (page[: Is * H].view(Is, H).contiguous(),
                           page[Is * H: 2 * Is * H].view(Is, H).contiguous(),
                           page[2 * Is * H:].view(H, Is).contiguous())

    @staticmethod
    def route(logits: torch.Tensor, top_k: int, renormalize: bool):
        p = torch.softmax(logits.to(torch.float32), dim=-1)
        order = torch.sort(p, dim=-1, descending=True, stable=True).indices[:, :top_k]
        w = torch.gather(p, 1, order)
        if renormalize:
            w = w / w.sum(dim=-1, keepdim=True)
        return w, order.to(torch.int32)

    def experts(self, x: torch.Tensor, w: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        """y [T, H] fp32 (values in the activation dtype) of the routed experts."""
        dt = self.dtype
        T, k = ids.shape
        c3 = torch.zeros((T, k, self.H), dtype=torch.float32)
        flat = ids.reshape(-1).to(torch.int64)
        order = torch.sort(flat, stable=True).indices
        sorted_ids = flat[order]
        experts, counts = torch.unique_consecutive(sorted_ids, return_counts=True)
        start = 0
        for e, c in zip(experts.tolist(), counts.tolist()):
            f = order[start:start + c]
            start += c
            if e not in self.w1:
                continue
            t, j = f // k, f % k
            xe = x[t]
            g = _round(xe @ self.w1[e].T, dt)
            u = _round(xe @ self.w3[e].T, dt)
            a = _round(_silu(g) * u, dt)
            c3[t, j] = _round((a @ self.w2[e].T) * w[t, j].unsqueeze(1), dt)
        y = c3[:, 0].clone()
        for j in range(1, k):
            y = y + c3[:, j]
        return _round(y, dt)

    def forward(self, x: torch.Tensor, logits: torch.Tensor, top_k: int, renormalize: bool,
                shared_gate: Optional[torch.Tensor] = None, scale: float = 1.0):
        """-> (y, w, ids): FusedMoE.forward on the host, plus the shared-expert block terms
        when the layer has a shared expert."""
        dt = self.dtype
        w, ids = self.route(logits, top_k, renormalize)
        y = self.experts(x, w, ids)
        if self.shared is None:
            return y, w, ids
        w1, w3, w2 = self.shared
        a = _round(_silu(_round(x @ w1.T, dt)) * _round(x @ w3.T, dt), dt)
        d = _round(a @ w2.T, dt)
        if shared_gate is not None:
            s = _round(torch.sigmoid(shared_gate.to(torch.float32).reshape(-1, 1)), dt)
            d = _round(s * d, dt)
        routed = _round(y * scale, dt) if scale != 1.0 else y
        return _round(routed + d, dt), w, ids
