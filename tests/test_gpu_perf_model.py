"""GPU smoke test of the performance-model refit: the operator harness profiles the fused MoE
at several token counts and the fitter produces a usable model."""
import pytest

from ae_amd.optimizer import GPUFusedMoEModel, PiecewiseLinearFitter
from ae_amd.optimizer.gpu_fused_moe_operator import GPUFusedMoEOperator, run_profile

pytestmark = pytest.mark.gpu


def test_profile_and_fit_small_operator():
    op = GPUFusedMoEOperator(num_experts=8, hidden_size=256, expert_size=256, top_k=2)
    x, s = op.create_dummy_input(16)
    y = op.forward(x, s)
    assert y.shape == (16, 256) and y.data_ptr() == x.data_ptr()
    prof = run_profile(op, [1, 2, 4, 8, 16, 32, 64, 128], num_warmup=1, num_runs=3)
    assert all(p["latency"] > 0 for p in prof)
    m = GPUFusedMoEModel(num_experts=8, hidden_size=256, expert_size=256, top_k=2)
    fit = PiecewiseLinearFitter(min_samples_per_segment=3).fit(m, prof)
    assert m.is_fitted and fit["num_samples"] == 8
    assert all(m.predict(n) >= 0 for n in (1, 50, 500))
