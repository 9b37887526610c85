"""GPU MoE latency model: two linear segments in the token count.

Reference: specmoe/optimizer/performance_simulator/models/gpu_fused_moe_model.py:11-47 (and
the BasePerformanceModel parameter handling, models/base.py). ``predict(N)`` is
``a1*N + b1`` for ``N <= breakpoint`` and ``a2*N + b2`` above, floored at 0, in seconds; it
feeds the solver's per-layer GPU time (specmoe/optimizer/solver.py:446-453).
"""
from __future__ import annotations

from typing import Any, Dict, List

import numpy as np


class GPUFusedMoEModel:
    def __init__(self, num_experts: int = 8, hidden_size: int = 4096, expert_size: int = 16384,
                 top_k: int = 2):
        self.name = "GPU_Fused_MoE_Piecewise"
        self.num_experts = num_experts
        self.hidden_size = hidden_size
        self.expert_size = expert_size
        self.top_k = top_k
        self.parameters: Dict[str, float] = {}
        self.is_fitted = False

    def set_parameters(self, parameters: Dict[str, float]) -> None:
        self.parameters = dict(parameters)
        self.is_fitted = True

    def get_parameters(self) -> Dict[str, float]:
        return dict(self.parameters)

    def get_parameter_names(self) -> List[str]:
        return ["a1", "b1", "a2", "b2", "breakpoint"]

    def predict(self, num_tokens: int, **kwargs) -> float:
        if not self.is_fitted:
            raise ValueError("the model has not been fitted")
        n = num_tokens
        if n <= self.parameters.get("breakpoint", 512):
            t = self.parameters["a1"] * n + self.parameters["b1"]
        else:
            t = self.parameters["a2"] * n + self.parameters["b2"]
        return max(0.0, t)

    def get_feature_vector(self, num_tokens: int, **kwargs) -> np.ndarray:
        return np.array([num_tokens, 1])

    def validate_input(self, num_tokens: int, **kwargs) -> bool:
        return num_tokens > 0

    def get_complexity_analysis(self, num_tokens: int, **kwargs) -> Dict[str, Any]:
        bp = self.parameters.get("breakpoint", 512) if self.is_fitted else 512
        left = num_tokens <= bp
        return {"regime": "Left Segment" if left else "Right Segment",
                "dominant_factor": "weight streaming (HBM)" if left else "token passes / compute",
                "breakpoint": bp, "token_count": num_tokens,
                "segment": f"{'Left' if left else 'Right'} segment"}
