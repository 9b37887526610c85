"""Drop-in MoE layer operators (the reference's specmoe/layers MoE surface)."""
from .FusedMoE import FusedMoE, UnquantizedFusedMoEMethod, set_weight_attrs
from .fused_moe_kernel import (fp32_gemm_outputs_fp16, fused_down_max_tokens, fused_moe_forward,
                               fused_moe_shared_forward, gateup_item_walk, gateup_waves,
                               moe_align_block_size, routing_in_gateup, set_fp32_gemm_outputs_fp16,
                               set_fused_down_max_tokens, set_gateup_item_walk, set_gateup_waves,
                               set_routing_in_gateup,
                               set_tiled_min_tokens, stack_fused_moe, stack_fused_moe_shared,
                               tiled_min_tokens)
from .layernorm import RMSNorm, add_rmsnorm_gate
from .mixtral_moe import MixtralMoE
from .moe_layer import PostAttentionMoE, moe_layer_forward
from .shared_moe import DeepseekV2MoE, Qwen2MoeSparseMoeBlock, SharedExpertMoE
from .topk import fused_topk, grouped_topk, select_experts

__all__ = [
    "FusedMoE", "UnquantizedFusedMoEMethod", "set_weight_attrs", "fused_moe_forward",
    "fused_moe_shared_forward", "moe_align_block_size", "stack_fused_moe",
    "stack_fused_moe_shared", "MixtralMoE",
    "SharedExpertMoE", "Qwen2MoeSparseMoeBlock", "DeepseekV2MoE", "fused_topk", "grouped_topk",
    "select_experts",
    "RMSNorm", "add_rmsnorm_gate", "PostAttentionMoE", "moe_layer_forward",
    "set_tiled_min_tokens", "tiled_min_tokens", "set_fused_down_max_tokens",
    "fused_down_max_tokens", "set_fp32_gemm_outputs_fp16", "fp32_gemm_outputs_fp16",
    "set_routing_in_gateup", "routing_in_gateup", "set_gateup_waves", "gateup_waves",
    "set_gateup_item_walk", "gateup_item_walk",
]
