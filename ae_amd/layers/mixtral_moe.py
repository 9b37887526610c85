"""The MoE block that calls FusedMoE: a drop-in for MixtralMoE.

Reference: specmoe/models/mixtral.py:59-115. ``forward(hidden_states, experts_mapping)``:
flatten to ``[T, H]``, router logits from a bias-free ``H -> E`` gate (a plain GEMM, left to
torch/hipBLASLt), FusedMoE over the expert pool page map, all-reduce across TP ranks when
TP > 1, restore the input shape. ``renormalize=True`` as in the reference.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from .FusedMoE import FusedMoE, _tp_rank_world


class MixtralMoE(nn.Module):
    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 params_dtype: Optional[torch.dtype] = None, quant_config=None,
                 tp_size: Optional[int] = None, prefix: str = "",
                 pin_experts_when_load_weight: bool = False):
        super().__init__()
        self.tp_size = _tp_rank_world()[1] if tp_size is None else tp_size
        self.hidden_size = hidden_size
        if params_dtype is None:
            params_dtype = torch.get_default_dtype()
        self.gate = nn.Linear(hidden_size, num_experts, bias=False, dtype=params_dtype)
        self.experts = FusedMoE(num_experts=num_experts, top_k=top_k, hidden_size=hidden_size,
                                intermediate_size=intermediate_size, params_dtype=params_dtype,
                                renormalize=True, quant_config=quant_config, tp_size=tp_size,
                                prefix=f"{prefix}.experts" if prefix else "experts",
                                pin_experts_when_load_weight=pin_experts_when_load_weight)

    def forward(self, hidden_states: torch.Tensor, experts_mapping: torch.Tensor) -> torch.Tensor:
        orig_shape = hidden_states.shape
        hidden_states = hidden_states.view(-1, self.hidden_size)
        router_logits = self.gate(hidden_states)
        final_hidden_states = self.experts(hidden_states, router_logits, experts_mapping)
        if self.tp_size > 1:
            torch.distributed.all_reduce(final_hidden_states)
        return final_hidden_states.view(orig_shape)
