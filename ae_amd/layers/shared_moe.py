"""MoE blocks with an always-active shared expert: Qwen1.5-MoE / Qwen2-MoE and DeepSeek-V2.

The reference serves only Mixtral (specmoe/models/mixtral.py:59-115) and has no shared expert.
These blocks put the public architectures' shared expert on the same routed path
(:class:`FusedMoE` over the pooled page cache, specmoe/layers/FusedMoE.py:155-196) and run
the whole block in one library call (``smx_fused_moe_shared_forward``):

- Qwen1.5-MoE-A2.7B: 60 routed experts (I 1408, top-4, no renormalisation) and one shared
  SwiGLU expert (I 5632) scaled by ``sigmoid(shared_expert_gate(x))``;
- DeepSeek-V2-Lite: 64 routed experts (I 1408, top-6, no renormalisation) and 2 shared
  experts, which form one SwiGLU MLP of 2*1408 columns, unscaled; the routed sum is
  multiplied by ``routed_scaling_factor`` (1.0 for V2-Lite). DeepSeek-V2 routes with the
  group-limited top-k (``n_group`` groups, ``topk_group`` selectable) and DeepSeek-V3 with the
  sigmoid top-k and a correction bias (``topk_method="noaux_tc"``): the grouped top-k
  (``smx_grouped_topk``), then the block on that routing (``smx_stack_fused_moe_shared``).

The shared expert's weights are packed like one pool page, ``[W1s | W3s | W2s]``
(``3*Is_p*H`` elements, ``Is_p = Is / tp``), and stay resident on the GPU: every token uses
them, so they are not offloaded.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from .FusedMoE import FusedMoE, _tp_rank_world
from .fused_moe_kernel import fused_moe_shared_forward, stack_fused_moe_shared
from .topk import grouped_topk, needs_grouped_topk


class SharedExpertMoE(nn.Module):
    """Router gate + FusedMoE + shared expert (+ optional shared-expert gate), one call.

    ``forward(hidden_states, experts_mapping)`` has MixtralMoE's signature: the routed
    experts' weights come from ``experts.ws.gpu_cache`` through ``experts_mapping``.
    """

    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 shared_intermediate_size: int, renormalize: bool, shared_expert_gate: bool,
                 routed_scaling_factor: float = 1.0, params_dtype: Optional[torch.dtype] = None,
                 tp_size: Optional[int] = None, prefix: str = "",
                 num_expert_group: Optional[int] = None, topk_group: Optional[int] = None,
                 correction_bias: bool = False):
        super().__init__()
        if params_dtype is None:
            params_dtype = torch.get_default_dtype()
        self.tp_size = _tp_rank_world()[1] if tp_size is None else tp_size
        assert shared_intermediate_size % self.tp_size == 0
        self.hidden_size = hidden_size
        self.top_k = top_k
        self.renormalize = renormalize
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.shared_size_per_partition = shared_intermediate_size // self.tp_size
        self.gate = nn.Linear(hidden_size, num_experts, bias=False, dtype=params_dtype)
        # grouped routing (select_experts' use_grouped_topk): groups, and the correction bias of
        # the sigmoid top-k, as the gate's e_score_correction_bias (fp32)
        self.num_expert_group = num_expert_group
        self.topk_group = topk_group
        if correction_bias:
            self.gate.e_score_correction_bias = nn.Parameter(
                torch.zeros(num_experts, dtype=torch.float32), requires_grad=False)
        self.use_grouped_topk = correction_bias or num_expert_group is not None
        self.shared_expert_gate = (nn.Linear(hidden_size, 1, bias=False, dtype=params_dtype)
                                   if shared_expert_gate else None)
        self.experts = FusedMoE(num_experts=num_experts, top_k=top_k, hidden_size=hidden_size,
                                intermediate_size=intermediate_size, params_dtype=params_dtype,
                                renormalize=renormalize, tp_size=self.tp_size,
                                prefix=f"{prefix}.experts" if prefix else "experts")
        self.shared_ws = nn.Parameter(
            torch.empty(3 * self.shared_size_per_partition * hidden_size, dtype=params_dtype),
            requires_grad=False)

    def load_shared_weights(self, gate_proj: torch.Tensor, up_proj: torch.Tensor,
                            down_proj: torch.Tensor) -> None:
        """Pack the shared MLP (gate/up ``[Is, H]``, down ``[H, Is]``) into ``shared_ws``:
        this TP rank's rows of gate and up, and its columns of down, as FusedMoE packs a
        routed expert's page."""
        rank = _tp_rank_world()[0] if self.tp_size > 1 else 0
        n = self.shared_size_per_partition
        H = self.hidden_size
        assert gate_proj.shape == up_proj.shape == (n * self.tp_size, H)
        assert down_proj.shape == (H, n * self.tp_size)
        shard = slice(rank * n, (rank + 1) * n)
        data = self.shared_ws.data
        data[0:n * H] = gate_proj[shard, :].reshape(-1)
        data[n * H:2 * n * H] = up_proj[shard, :].reshape(-1)
        data[2 * n * H:] = down_proj[:, shard].reshape(-1)

    def forward(self, hidden_states: torch.Tensor, experts_mapping: torch.Tensor) -> torch.Tensor:
        orig_shape = hidden_states.shape
        hidden_states = hidden_states.view(-1, self.hidden_size)
        router_logits = self.gate(hidden_states)
        sgate = self.shared_expert_gate(hidden_states) if self.shared_expert_gate is not None else None
        pool = getattr(self.experts.ws, "gpu_cache", None)
        if pool is None:
            raise RuntimeError("no expert pool attached: set experts.ws.gpu_cache before forward")
        bias = getattr(self.gate, "e_score_correction_bias", None)
        ng = self.num_expert_group or 1
        tg = self.topk_group or ng
        if needs_grouped_topk(self.use_grouped_topk, tg, ng, bias):
            w, ids = grouped_topk(router_logits, self.top_k, self.renormalize, ng, tg, bias)
            out = stack_fused_moe_shared(hidden_states, pool, experts_mapping, w, ids,
                                         self.shared_ws.data, sgate, self.routed_scaling_factor,
                                         inplace=True)
        else:
            out = fused_moe_shared_forward(hidden_states, router_logits, pool, experts_mapping,
                                           self.top_k, self.renormalize, self.shared_ws.data,
                                           sgate, self.routed_scaling_factor, inplace=True)
        if self.tp_size > 1:
            torch.distributed.all_reduce(out)
        return out.view(orig_shape)


class Qwen2MoeSparseMoeBlock(SharedExpertMoE):
    """Qwen1.5-MoE / Qwen2-MoE block: gated shared expert, no top-k renormalisation
    (``norm_topk_prob = False``)."""

    def __init__(self, num_experts: int = 60, top_k: int = 4, hidden_size: int = 2048,
                 moe_intermediate_size: int = 1408, shared_expert_intermediate_size: int = 5632,
                 norm_topk_prob: bool = False, params_dtype: Optional[torch.dtype] = None,
                 tp_size: Optional[int] = None, prefix: str = ""):
        super().__init__(num_experts, top_k, hidden_size, moe_intermediate_size,
                         shared_expert_intermediate_size, renormalize=norm_topk_prob,
                         shared_expert_gate=True, params_dtype=params_dtype, tp_size=tp_size,
                         prefix=prefix)


class DeepseekV2MoE(SharedExpertMoE):
    """DeepSeek-V2 block: ungated shared experts fused into one MLP of
    ``n_shared_experts * moe_intermediate_size`` columns, routed output scaled by
    ``routed_scaling_factor``. Routing by ``topk_method``: "greedy" (top-k softmax, one group:
    DeepSeek-V2-Lite), "group_limited_greedy" (softmax, the ``topk_group`` best of ``n_group``
    expert groups: DeepSeek-V2) or "noaux_tc" (sigmoid scores plus the gate's
    ``e_score_correction_bias`` choose, group-limited: DeepSeek-V3)."""

    def __init__(self, n_routed_experts: int = 64, num_experts_per_tok: int = 6,
                 hidden_size: int = 2048, moe_intermediate_size: int = 1408,
                 n_shared_experts: int = 2, routed_scaling_factor: float = 1.0,
                 norm_topk_prob: bool = False, params_dtype: Optional[torch.dtype] = None,
                 tp_size: Optional[int] = None, prefix: str = "", topk_method: str = "greedy",
                 n_group: int = 1, topk_group: int = 1):
        if topk_method not in ("greedy", "group_limited_greedy", "noaux_tc"):
            raise ValueError(f"unknown topk_method {topk_method!r}")
        grouped = topk_method != "greedy"
        super().__init__(n_routed_experts, num_experts_per_tok, hidden_size,
                         moe_intermediate_size, n_shared_experts * moe_intermediate_size,
                         renormalize=norm_topk_prob, shared_expert_gate=False,
                         routed_scaling_factor=routed_scaling_factor, params_dtype=params_dtype,
                         tp_size=tp_size, prefix=prefix,
                         num_expert_group=n_group if grouped else None,
                         topk_group=topk_group if grouped else None,
                         correction_bias=topk_method == "noaux_tc")
