"""The MoE operator the solver's model is fit to, and its profiler.

Reference: specmoe/optimizer/performance_simulator/operators/gpu_fused_moe.py:15-95 (a
FusedMoE over a 2E-slot fp16 pool mapped through [0,2,3,6,8,10,12,14], random fp16 tokens and
scores) and profiler/operator_profiler.py:16-150 (warm-up, then the mean latency of
``num_runs`` forwards). Latency here is device time from HIP events around the runs.
"""
from __future__ import annotations

import time
from typing import Any, Dict, List

import torch

from ..layers import FusedMoE, set_weight_attrs


class GPUFusedMoEOperator:
    def __init__(self, num_experts: int = 8, expert_capacity: int = None, hidden_size: int = 4096,
                 expert_size: int = 16384, top_k: int = 2, dtype: torch.dtype = torch.float16):
        self.name = "GPU_Fused_MoE"
        self.num_experts = num_experts
        self.hidden_size = hidden_size
        self.expert_size = expert_size
        self.top_k = top_k
        self.dtype = dtype
        pool = torch.ones((2 * num_experts, 3 * hidden_size * expert_size), device="cuda", dtype=dtype)
        self.indices = torch.arange(0, 2 * num_experts, 2, dtype=torch.int64, device="cuda")
        if num_experts == 8:
            self.indices = torch.tensor([0, 2, 3, 6, 8, 10, 12, 14], dtype=torch.int64, device="cuda")
        self.fused_moe = FusedMoE(num_experts=num_experts, top_k=top_k, hidden_size=hidden_size,
                                  intermediate_size=expert_size, params_dtype=dtype, tp_size=1)
        set_weight_attrs(self.fused_moe.ws, {"gpu_cache": pool})

    def forward(self, input_tokens: torch.Tensor, score: torch.Tensor, **kwargs) -> torch.Tensor:
        return self.fused_moe(input_tokens, score, self.indices)

    def create_dummy_input(self, num_tokens: int = 1024):
        return (torch.randn(num_tokens, self.hidden_size, device="cuda", dtype=self.dtype),
                torch.randn(num_tokens, self.num_experts, device="cuda", dtype=self.dtype))

    def get_flops(self, num_tokens: int = 1024, **kwargs) -> int:
        return 2 * num_tokens * self.top_k * 3 * self.hidden_size * self.expert_size


def run_profile(operator: GPUFusedMoEOperator, token_counts: List[int], num_warmup: int = 2,
                num_runs: int = 10) -> List[Dict[str, Any]]:
    """[{'input_params': {'num_tokens': N}, 'latency': seconds per forward}] -- the profile
    record format the fitter reads."""
    results = []
    stream = torch.cuda.current_stream()
    for n in token_counts:
        x, s = operator.create_dummy_input(n)
        for _ in range(num_warmup):
            operator.forward(x.clone(), s)
        xs = [x.clone() for _ in range(num_runs)]  # forward writes its input in place
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(num_runs):
            operator.forward(xs[i], s)
        b.record(stream)
        torch.cuda.synchronize()
        results.append({"input_params": {"num_tokens": int(n)},
                        "latency": a.elapsed_time(b) / 1000.0 / num_runs,
                        "num_runs": num_runs, "timestamp": time.time()})
    return results
