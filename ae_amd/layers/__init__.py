"""Drop-in MoE layer operators (the reference's specmoe/layers MoE surface)."""
from .FusedMoE import FusedMoE, UnquantizedFusedMoEMethod, set_weight_attrs
from .fused_moe_kernel import fused_moe_forward, moe_align_block_size, stack_fused_moe
from .mixtral_moe import MixtralMoE
from .topk import fused_topk, select_experts

__all__ = [
    "FusedMoE", "UnquantizedFusedMoEMethod", "set_weight_attrs", "fused_moe_forward",
    "moe_align_block_size", "stack_fused_moe", "MixtralMoE", "fused_topk", "select_experts",
]
