"""Top-k softmax routing: the `select_experts` the reference's MoE layer calls.

Reference call site: specmoe/layers/FusedMoE.py:174-185, which calls
``sglang.srt.layers.moe.topk.select_experts`` (sglang==0.4.5.post3, not vendored). Its
dispatch, kept here:

- ``use_grouped_topk``: the grouped top-k (``smx_grouped_topk``). The experts form
  ``num_expert_group`` groups of consecutive experts, only the ``topk_group`` best groups are
  selectable. Without ``correction_bias`` (sglang's ``grouped_topk``): softmax scores, a
  group ranks by its best score. With it (``biased_grouped_topk``): sigmoid scores, experts
  and groups rank by score + bias (a group by the sum of its two best), the weights are the
  unbiased scores. A custom routing function is not called on this branch.
- otherwise ``fused_topk``: an fp32 softmax over the experts (sgl_kernel.topk_softmax), top-k
  in descending order with ties resolved to the lower expert index (``smx_topk_softmax``);
  ``correction_bias`` is not used on this branch.
- a ``custom_routing_function`` replaces ``fused_topk``: it is called as
  ``custom_routing_function(hidden_states=..., gating_output=..., topk=..., renormalize=...)``
  and its ``(weights, ids)`` are returned as fp32 / int32.

Each branch renormalises ``w / w.sum(-1)`` when asked. Returns ``(topk_weights fp32 [T,k],
topk_ids int32 [T,k])``. Where sglang's ``torch.topk(sorted=False)`` leaves the order of the
picks open, they come in descending order here (ties to the lower index), as from
``fused_topk``.

``routed_scaling_factor`` is accepted and changes no weight: sglang 0.4.5.post3's
``select_experts`` hands it only to its grouped top-k, where it sets the weight of a shared
expert fused into the top-k (``topk_weights[:, -1] =
topk_weights[:, :-1].sum(-1) / routed_scaling_factor``, and only when the server's
``n_share_experts_fusion`` is set, which defaults to 0); the ungrouped ``fused_topk`` and a
custom routing function never see it. Scaling the routed output by the factor is the model
block's job (DeepSeek-V2's MoE multiplies its routed output by it), which this build does in
the block entry points (``fused_moe_shared_forward``, ``moe_layer_forward``). The reference
itself never sets the factor (specmoe/layers/FusedMoE.py:287 defaults it to None and passes it
through at :184,298,526). Parity with sglang is unpinned here: it is not vendored.
"""
from __future__ import annotations

import math
from typing import Callable, Optional, Tuple

import torch

from .. import _lib
from ._torch import dtype_code, ptr, require_gpu, stream_of


def check_routing_options(use_grouped_topk: bool, topk_group: Optional[int],
                          num_expert_group: Optional[int],
                          custom_routing_function: Optional[Callable],
                          correction_bias: Optional[torch.Tensor],
                          routed_scaling_factor: Optional[float]) -> None:
    """select_experts' checks: the grouped top-k needs both group sizes (sglang asserts them);
    routed_scaling_factor is accepted (it does not change the weights of these selections,
    see the module docstring) but must be finite."""
    if use_grouped_topk and (topk_group is None or num_expert_group is None):
        raise ValueError("grouped top-k needs topk_group and num_expert_group")
    if routed_scaling_factor is not None and not math.isfinite(float(routed_scaling_factor)):
        raise ValueError(f"routed_scaling_factor must be finite, got {routed_scaling_factor}")


def needs_grouped_topk(use_grouped_topk: bool, topk_group: Optional[int],
                       num_expert_group: Optional[int],
                       correction_bias: Optional[torch.Tensor]) -> bool:
    """Whether select_experts must run the grouped top-k. Without a bias, one group or every
    group selectable is the plain top-k (same softmax, same picks in the same order, same
    weights), which the one-call MoE entry points run themselves."""
    if not use_grouped_topk:
        return False
    return correction_bias is not None or not (num_expert_group == 1 or topk_group == num_expert_group)


def grouped_topk(router_logits: torch.Tensor, top_k: int, renormalize: bool,
                 num_expert_group: int, topk_group: int,
                 correction_bias: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """sglang's grouped_topk / biased_grouped_topk on the GPU (``smx_grouped_topk``); the
    bias is read as fp32 (sglang adds it to fp32 scores, which promotes it the same way)."""
    require_gpu(router_logits)
    logits = router_logits.contiguous()
    T, E = logits.shape
    bias = None
    if correction_bias is not None:
        if correction_bias.numel() != E:
            raise ValueError(f"correction_bias has {correction_bias.numel()} values for {E} experts")
        bias = correction_bias.to(device=logits.device, dtype=torch.float32).contiguous()
    w = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    _lib.call("smx_grouped_topk", ptr(logits), dtype_code(logits.dtype), T, E, top_k,
              int(bool(renormalize)), int(num_expert_group), int(topk_group),
              ptr(bias) if bias is not None else None, ptr(w), ptr(ids), stream_of(logits))
    return w, ids


def select_experts(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    top_k: int,
    use_grouped_topk: bool = False,
    renormalize: bool = True,
    topk_group: Optional[int] = None,
    num_expert_group: Optional[int] = None,
    custom_routing_function: Optional[Callable] = None,
    correction_bias: Optional[torch.Tensor] = None,
    torch_native: bool = False,
    routed_scaling_factor: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    check_routing_options(use_grouped_topk, topk_group, num_expert_group,
                          custom_routing_function, correction_bias, routed_scaling_factor)
    if use_grouped_topk:
        assert hidden_states.shape[0] == router_logits.shape[0], "Number of tokens mismatch"
        return grouped_topk(router_logits, top_k, renormalize, num_expert_group, topk_group,
                            correction_bias)
    if custom_routing_function is not None:
        w, ids = custom_routing_function(hidden_states=hidden_states, gating_output=router_logits,
                                         topk=top_k, renormalize=renormalize)
        return w.to(torch.float32), ids.to(torch.int32)
    if torch_native:
        raise NotImplementedError("torch_native routing (this build routes on the GPU only)")
    assert hidden_states.shape[0] == router_logits.shape[0], "Number of tokens mismatch"
    require_gpu(router_logits)
    logits = router_logits.contiguous()
    T, E = logits.shape
    w = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    _lib.call("smx_topk_softmax", ptr(logits), dtype_code(logits.dtype), T, E, top_k,
              int(bool(renormalize)), ptr(w), ptr(ids), stream_of(logits))
    return w, ids


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int,
               renormalize: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """sglang's fused_topk (the ungrouped branch select_experts dispatches to)."""
    return select_experts(hidden_states, gating_output, topk, False, renormalize)
