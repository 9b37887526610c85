"""The post-attention half of a MoE decoder layer in one library call.

Reference: the sequence at specmoe/models/mixtral.py:310-313 -- ``hidden, residual =
post_attention_layernorm(hidden, residual)`` (RMSNorm with fused residual add,
specmoe/layers/layernorm.py:23-33) then ``hidden = block_sparse_moe(hidden,
experts_mapping)`` (MixtralMoE.forward, :106-115: router gate, FusedMoE). Here the residual
add, the norm, the router gate and the top-k run in one kernel, followed by the expert sort,
the expert kernels and the combine (smx_moe_layer_forward). Blocks with a shared expert
(SharedExpertMoE) run the same way, their shared-expert gate as one more router row. A block
whose routing is not the plain top-k softmax (grouped top-k, a correction bias, a custom routing
function) runs as the norm and then the block, two calls.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import nn

from .. import _lib
from ._torch import dtype_code, ptr, require_gpu, stream_of, workspace
from .fused_moe_kernel import _as_index, _pool_geometry
from .layernorm import RMSNorm
from .mixtral_moe import MixtralMoE
from .shared_moe import SharedExpertMoE
from .topk import needs_grouped_topk


def moe_layer_forward(hidden: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                      eps: float, gate_weight: torch.Tensor, w1: torch.Tensor,
                      indicies: torch.Tensor, top_k: int, renormalize: bool,
                      shared_w: Optional[torch.Tensor] = None,
                      shared_gate_weight: Optional[torch.Tensor] = None,
                      routed_scaling_factor: float = 1.0, return_routing: bool = False):
    """residual <- hidden + residual; hidden <- MoE(RMSNorm(residual)), all in place.

    ``gate_weight`` ``[E, H]``; ``w1`` the expert pool ``[P, 3*I*H]`` with ``indicies`` the
    expert -> slot map; ``shared_w`` an optional shared-expert page ``[3*Is*H]`` and
    ``shared_gate_weight`` its optional gate row ``[H]``. Returns ``hidden`` (and
    ``(router_logits, topk_weights, topk_ids)`` with ``return_routing``)."""
    assert hidden.dim() == 2 and hidden.is_contiguous(), "hidden states must be [T, H] contiguous"
    require_gpu(hidden, residual, norm_weight, gate_weight, w1, indicies, shared_w, shared_gate_weight)
    T, H = hidden.shape
    H_, I = _pool_geometry(hidden, w1)
    E = gate_weight.shape[0]
    for t in (residual, norm_weight, gate_weight, w1, shared_w, shared_gate_weight):
        if t is not None:
            assert t.dtype == hidden.dtype and t.is_contiguous(), "dtype/contiguity mismatch"
    Is = 0
    if shared_w is not None:
        assert shared_w.numel() % (3 * H) == 0, "shared expert page is not 3*Is*H elements"
        Is = shared_w.numel() // (3 * H)
    dt = dtype_code(hidden.dtype)
    nbytes = _lib.lib().smx_moe_layer_workspace_size(T, H, I, E, top_k, Is, dt)
    if nbytes == 0 and T > 0:
        raise ValueError(f"unsupported MoE layer shape T={T} H={H} I={I} E={E} top_k={top_k} "
                         f"shared I={Is}")
    ws = workspace(nbytes, hidden.device)
    slots = _as_index(indicies, torch.int64)
    logits = w = ids = None
    if return_routing:
        logits = torch.empty((T, E), dtype=hidden.dtype, device=hidden.device)
        w = torch.empty((T, top_k), dtype=torch.float32, device=hidden.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=hidden.device)
    _lib.call("smx_moe_layer_forward", ptr(hidden), ptr(residual), dt, T, H, ptr(norm_weight),
              float(eps), ptr(gate_weight), E, top_k, int(bool(renormalize)), ptr(w1), w1.shape[0],
              w1.shape[1], ptr(slots), ptr(shared_w), Is, ptr(shared_gate_weight),
              float(routed_scaling_factor), ptr(logits), ptr(w), ptr(ids), ptr(ws), ws.numel(),
              stream_of(hidden))
    if return_routing:
        return hidden, (logits, w, ids)
    return hidden


class PostAttentionMoE(nn.Module):
    """``post_attention_layernorm`` + ``block_sparse_moe`` of a decoder layer as one call.

    ``forward(hidden_states, residual, experts_mapping) -> (hidden_states, residual)``, the
    pair the reference's decoder layer returns after its MoE (mixtral.py:310-315). The
    modules keep their own parameters (and weight loading); only the execution is fused.
    """

    def __init__(self, layernorm: RMSNorm, block: nn.Module):
        super().__init__()
        if not isinstance(block, (MixtralMoE, SharedExpertMoE)):
            raise TypeError("block must be MixtralMoE or SharedExpertMoE")
        self.post_attention_layernorm = layernorm
        self.block_sparse_moe = block

    @staticmethod
    def _grouped_routing(blk: nn.Module) -> bool:
        if isinstance(blk, SharedExpertMoE):
            ng = blk.num_expert_group or 1
            return needs_grouped_topk(blk.use_grouped_topk, blk.topk_group or ng, ng,
                                      getattr(blk.gate, "e_score_correction_bias", None))
        ex = blk.experts
        return ex.custom_routing_function is not None or needs_grouped_topk(
            ex.use_grouped_topk, ex.topk_group, ex.num_expert_group, ex.correction_bias)

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor,
                experts_mapping: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        blk = self.block_sparse_moe
        shape = hidden_states.shape
        H = shape[-1]
        h2 = hidden_states.view(-1, H)
        pool = getattr(blk.experts.ws, "gpu_cache", None)
        if pool is None:
            raise RuntimeError("no expert pool attached: set experts.ws.gpu_cache before forward")
        if self._grouped_routing(blk):
            # the fused call's top-k is the plain one: the norm (residual add in place), then
            # the block with its grouped top-k (select_experts' use_grouped_topk branch)
            xs, _ = self.post_attention_layernorm(h2, residual.view(-1, H))
            blk(xs, experts_mapping)
            return hidden_states, residual
        nw = self.post_attention_layernorm.weight.data
        if nw.dtype != h2.dtype:
            nw = nw.to(h2.dtype)
        shared = isinstance(blk, SharedExpertMoE)
        moe_layer_forward(
            h2, residual.view(-1, H), nw, self.post_attention_layernorm.variance_epsilon,
            blk.gate.weight.data, pool, experts_mapping, blk.experts.top_k,
            blk.experts.renormalize,
            shared_w=blk.shared_ws.data if shared else None,
            shared_gate_weight=(blk.shared_expert_gate.weight.data.view(-1)
                                if shared and blk.shared_expert_gate is not None else None),
            routed_scaling_factor=blk.routed_scaling_factor if shared else 1.0)
        if blk.tp_size > 1:
            torch.distributed.all_reduce(h2)
        return hidden_states, residual
