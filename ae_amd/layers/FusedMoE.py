"""FusedMoE layer on MI355X: a drop-in for specmoe/layers/FusedMoE.py.

Same constructor arguments, the same ``ws`` parameter protocol (master weights
``[E, 3*I_p*H]`` on the host, the GPU pool attached by the engine as ``ws.gpu_cache``), the
same weight_loader page packing, and the same
``forward(hidden_states, router_logits, expert_cache_indices)``; the computation runs in
libspecmoe_mi355x.so. Routing options that would select different experts than the plain
top-k (grouped top-k over several groups, a correction bias) raise NotImplementedError
instead of silently computing something else. The options the reference's forward_cuda
accepts and ignores -- ``activation``, ``apply_router_weight_on_input``, ``inplace`` and
``no_combine`` (specmoe/layers/FusedMoE.py:155-196 always runs SiLU, weights after the down
projection, combines and writes in place) -- are accepted and ignored the same way, with a
one-time warning for a non-default value.
"""
from __future__ import annotations

import warnings
from enum import Enum
from typing import Callable, List, Optional, Tuple

import torch

from .fused_moe_kernel import fused_moe_forward, stack_fused_moe
from .topk import check_routing_options, needs_grouped_topk, select_experts


def _tp_rank_world() -> Tuple[int, int]:
    """Tensor-parallel rank/size: the default process group when initialised, else (0, 1)."""
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        return torch.distributed.get_rank(), torch.distributed.get_world_size()
    return 0, 1


def set_weight_attrs(weight: torch.Tensor, weight_attrs: Optional[dict]) -> None:
    """Attach attributes to a parameter (the engine attaches the GPU pool as ``gpu_cache``)."""
    if weight_attrs is None:
        return
    for key, value in weight_attrs.items():
        setattr(weight, key, value)


# Options forward_cuda ignores, as the reference's does, and their default values.
_IGNORED_DEFAULTS = {"activation": "silu", "apply_router_weight_on_input": False,
                     "inplace": True, "no_combine": False}
_warned: set = set()


def warn_ignored_options(**values) -> None:
    """Warn once per (option, value) when an option the reference ignores is not its
    default: the result is the SiLU, combined, in-place output regardless."""
    for name, value in values.items():
        if value != _IGNORED_DEFAULTS[name] and (name, repr(value)) not in _warned:
            _warned.add((name, repr(value)))
            warnings.warn(f"FusedMoE: {name}={value!r} is ignored, as in the reference's "
                          "forward_cuda (SiLU, routing weights after the down projection, "
                          "combined, in place)", RuntimeWarning, stacklevel=3)


class FusedMoeWeightScaleSupported(Enum):
    TENSOR = "tensor"
    CHANNEL = "channel"
    GROUP = "group"
    BLOCK = "block"


class UnquantizedFusedMoEMethod:
    """Unquantized MoE method. Reference: specmoe/layers/FusedMoE.py:65-240."""

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size: int, params_dtype: torch.dtype, **extra_weight_attrs):
        """``ws``: ``[E, 3*I*H]`` on the host, pinned when the layer asks for it
        (reference :68-96; pinned allocation is hipHostMalloc through torch here)."""
        shape = (num_experts, 3 * intermediate_size * hidden_size)
        if layer.pin_experts_when_load_weight:
            if not torch.cuda.is_available():
                raise RuntimeError("pin_experts_when_load_weight needs a GPU for pinned host memory")
            data = torch.empty(shape, dtype=params_dtype, device="cpu", pin_memory=True)
        else:
            data = torch.empty(shape, dtype=params_dtype, device="cpu")
        ws_weight = torch.nn.Parameter(data, requires_grad=False)
        layer.register_parameter("ws", ws_weight)
        extra_weight_attrs.pop("intermediate_size_per_partition", None)
        set_weight_attrs(ws_weight, extra_weight_attrs)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, router_logits: torch.Tensor,
              expert_cache_indices: torch.Tensor, top_k: int, renormalize: bool,
              use_grouped_topk: bool, topk_group: Optional[int] = None,
              num_expert_group: Optional[int] = None,
              custom_routing_function: Optional[Callable] = None,
              correction_bias: Optional[torch.Tensor] = None, activation: str = "silu",
              apply_router_weight_on_input: bool = False, inplace: bool = True,
              no_combine: bool = False,
              routed_scaling_factor: Optional[float] = None) -> torch.Tensor:
        return self.forward_cuda(
            layer=layer, x=x, expert_cache_indices=expert_cache_indices,
            use_grouped_topk=use_grouped_topk, top_k=top_k, router_logits=router_logits,
            renormalize=renormalize, topk_group=topk_group, num_expert_group=num_expert_group,
            custom_routing_function=custom_routing_function, correction_bias=correction_bias,
            activation=activation, apply_router_weight_on_input=apply_router_weight_on_input,
            inplace=inplace, no_combine=no_combine, routed_scaling_factor=routed_scaling_factor)

    def forward_cuda(self, layer: torch.nn.Module, x: torch.Tensor,
                     expert_cache_indices: torch.Tensor, use_grouped_topk: bool, top_k: int,
                     router_logits: torch.Tensor, renormalize: bool,
                     topk_group: Optional[int] = None, num_expert_group: Optional[int] = None,
                     custom_routing_function: Optional[Callable] = None,
                     correction_bias: Optional[torch.Tensor] = None, activation: str = "silu",
                     apply_router_weight_on_input: bool = False, inplace: bool = True,
                     no_combine: bool = False,
                     routed_scaling_factor: Optional[float] = None) -> torch.Tensor:
        """Reference :155-196: select_experts, then stack_fused_moe(inplace=True) on the
        pool ``layer.ws.gpu_cache`` -- here one library call."""
        check_routing_options(use_grouped_topk, topk_group, num_expert_group,
                              custom_routing_function, correction_bias, routed_scaling_factor)
        warn_ignored_options(activation=activation,
                             apply_router_weight_on_input=apply_router_weight_on_input,
                             inplace=inplace, no_combine=no_combine)
        pool = getattr(layer.ws, "gpu_cache", None)
        if pool is None:
            raise RuntimeError("no expert pool attached: set ws.gpu_cache before forward")
        if custom_routing_function is not None or needs_grouped_topk(
                use_grouped_topk, topk_group, num_expert_group, correction_bias):
            # a caller's routing or the grouped top-k, then the experts on the pool
            # (reference :174-196)
            topk_weights, topk_ids = select_experts(
                x, router_logits, top_k, use_grouped_topk, renormalize, topk_group=topk_group,
                num_expert_group=num_expert_group,
                custom_routing_function=custom_routing_function,
                correction_bias=correction_bias, routed_scaling_factor=routed_scaling_factor)
            return stack_fused_moe(x, pool, expert_cache_indices, router_logits, topk_weights,
                                   topk_ids, renormalize, inplace=True)
        return fused_moe_forward(x, router_logits, pool, expert_cache_indices, top_k,
                                 renormalize, inplace=True)

    def forward_cpu(self, *args, **kwargs) -> torch.Tensor:
        raise NotImplementedError("this build has no CPU MoE path")

    def forward_tpu(self, *args, **kwargs) -> torch.Tensor:
        raise NotImplementedError("The TPU backend currently does not support MoE.")

    forward_native = forward_cuda


class FusedMoE(torch.nn.Module):
    """FusedMoE layer. Reference: specmoe/layers/FusedMoE.py:243-593.

    Args are the reference's (:265-289). ``quant_config`` must be None (the unquantized
    method is the only one built); ``reduce_results`` all-reduces over the default process
    group when the TP size is above 1.
    """

    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 params_dtype: Optional[torch.dtype] = None, reduce_results: bool = False,
                 renormalize: bool = True, use_grouped_topk: bool = False,
                 num_expert_group: Optional[int] = None, topk_group: Optional[int] = None,
                 quant_config=None, tp_size: Optional[int] = None, prefix: str = "",
                 custom_routing_function: Optional[Callable] = None,
                 correction_bias: Optional[torch.Tensor] = None, activation: str = "silu",
                 apply_router_weight_on_input: bool = False, use_presharded_weights: bool = False,
                 inplace: bool = True, no_combine: bool = False,
                 routed_scaling_factor: Optional[float] = None,
                 pin_experts_when_load_weight: bool = False):
        super().__init__()
        if params_dtype is None:
            params_dtype = torch.get_default_dtype()
        self.tp_size = tp_size if tp_size is not None else _tp_rank_world()[1]
        self.routed_scaling_factor = routed_scaling_factor
        self.top_k = top_k
        self.num_experts = num_experts
        assert intermediate_size % self.tp_size == 0
        self.intermediate_size_per_partition = intermediate_size // self.tp_size
        self.hidden_size = hidden_size
        self.reduce_results = reduce_results
        self.renormalize = renormalize
        self.use_grouped_topk = use_grouped_topk
        if self.use_grouped_topk:
            assert num_expert_group is not None and topk_group is not None
        self.num_expert_group = num_expert_group
        self.topk_group = topk_group
        self.custom_routing_function = custom_routing_function
        self.correction_bias = correction_bias
        self.activation = activation
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self.use_presharded_weights = use_presharded_weights
        self.inplace = inplace
        self.no_combine = no_combine
        self.local_num_experts = num_experts
        self.pin_experts_when_load_weight = pin_experts_when_load_weight
        if quant_config is not None:
            raise NotImplementedError("quantized MoE methods")
        self.quant_method = UnquantizedFusedMoEMethod()
        self.quant_method.create_weights(
            layer=self, num_experts=num_experts, hidden_size=hidden_size,
            intermediate_size=self.intermediate_size_per_partition,
            intermediate_size_per_partition=self.intermediate_size_per_partition,
            params_dtype=params_dtype, weight_loader=self.weight_loader)

    def weight_loader(self, param: torch.nn.Parameter, loaded_weight: torch.Tensor,
                      weight_name: str, shard_id: str, expert_id: int) -> None:
        """Pack one HF expert matrix into its page (reference :485-505): w1 (gate, [I,H])
        rows of this TP shard at [0, I_p*H), w3 (up) at [I_p*H, 2*I_p*H), and the shard's
        columns of w2 (down, [H,I]) at [2*I_p*H, 3*I_p*H)."""
        tp_rank = _tp_rank_world()[0] if self.tp_size > 1 else 0
        param_data = param.data
        shard_size = self.intermediate_size_per_partition
        shard = slice(tp_rank * shard_size, (tp_rank + 1) * shard_size)
        w3_offset = shard_size * self.hidden_size
        w2_offset = 2 * shard_size * self.hidden_size
        if weight_name.endswith("w1.weight"):
            param_data[expert_id, 0:w3_offset] = loaded_weight[shard, :].reshape(-1)
        if weight_name.endswith("w3.weight"):
            param_data[expert_id, w3_offset:w2_offset] = loaded_weight[shard, :].reshape(-1)
        if weight_name.endswith("w2.weight"):
            param_data[expert_id, w2_offset:] = loaded_weight[:, shard].reshape(-1)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor,
                expert_cache_indices: torch.Tensor) -> torch.Tensor:
        """Reference :508-532. Writes the result into hidden_states and returns it."""
        final_hidden_states = self.quant_method.apply(
            layer=self, x=hidden_states, router_logits=router_logits,
            expert_cache_indices=expert_cache_indices, top_k=self.top_k,
            renormalize=self.renormalize, use_grouped_topk=self.use_grouped_topk,
            topk_group=self.topk_group, num_expert_group=self.num_expert_group,
            custom_routing_function=self.custom_routing_function,
            correction_bias=self.correction_bias, activation=self.activation,
            apply_router_weight_on_input=self.apply_router_weight_on_input,
            routed_scaling_factor=self.routed_scaling_factor)
        if self.reduce_results and self.tp_size > 1:
            torch.distributed.all_reduce(final_hidden_states)
        return final_hidden_states

    @classmethod
    def make_expert_params_mapping(cls, ckpt_gate_proj_name: str, ckpt_down_proj_name: str,
                                   ckpt_up_proj_name: str,
                                   num_experts: int) -> List[Tuple[str, str, int, str]]:
        """(param_name, weight_name, expert_id, shard_id) per checkpoint tensor (ref :534-559)."""
        return [
            ("experts.ws", f"experts.{expert_id}.{weight_name}.weight", expert_id, shard_id)
            for expert_id in range(num_experts)
            for shard_id, weight_name in [
                ("w1", ckpt_gate_proj_name),
                ("w2", ckpt_down_proj_name),
                ("w3", ckpt_up_proj_name),
            ]
        ]
