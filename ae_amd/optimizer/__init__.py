"""The solver's MoE performance model, re-fit on MI355X (the reference's
specmoe/optimizer/performance_simulator: GPUFusedMoEModel, its operator harness, profiler
and piecewise-linear fitter), measuring this library's MoE kernels."""
from .gpu_fused_moe_model import GPUFusedMoEModel
from .piecewise_fitter import PiecewiseLinearFitter

__all__ = ["GPUFusedMoEModel", "PiecewiseLinearFitter"]
