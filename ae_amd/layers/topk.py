"""Top-k softmax routing: the `select_experts` the reference's MoE layer calls.

Reference call site: specmoe/layers/FusedMoE.py:174-185, which calls
``sglang.srt.layers.moe.topk.select_experts`` (sglang==0.4.5.post3, not vendored): an fp32
softmax over the experts (sgl_kernel.topk_softmax), top-k selection in descending order
with ties resolved to the lower expert index, then an optional renormalisation
``w / w.sum(-1)``. Returns ``(topk_weights fp32 [T,k], topk_ids int32 [T,k])``. A
``custom_routing_function`` replaces that selection: it is called as
``custom_routing_function(hidden_states=..., gating_output=..., topk=..., renormalize=...)``
and its ``(weights, ids)`` are returned as fp32 / int32.

``routed_scaling_factor`` is accepted and, on the paths this build takes, changes nothing:
sglang 0.4.5.post3's ``select_experts`` hands it only to its grouped top-k, where it sets
the weight of a shared expert fused into the top-k (``topk_weights[:, -1] =
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
    """Reject the select_experts options this build does not implement.

    Grouped top-k with a single group is plain top-k and is accepted; a custom routing
    function is called as the reference calls it; routed_scaling_factor is accepted (it does
    not change the weights of these selections, see the module docstring) but must be finite.
    """
    if use_grouped_topk and not (num_expert_group in (None, 1) and topk_group in (None, 1)):
        raise NotImplementedError("grouped top-k with more than one expert group")
    if custom_routing_function is not None and use_grouped_topk:
        raise NotImplementedError("custom_routing_function together with grouped top-k")
    if correction_bias is not None:
        raise NotImplementedError("correction_bias (biased grouped top-k)")
    if routed_scaling_factor is not None and not math.isfinite(float(routed_scaling_factor)):
        raise ValueError(f"routed_scaling_factor must be finite, got {routed_scaling_factor}")


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
