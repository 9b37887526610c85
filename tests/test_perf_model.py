"""CPU tests of the MoE performance model and its piecewise-linear fitter (the solver's
GPUFusedMoEModel refit): exact recovery, agreement with scikit-learn's least squares, the
breakpoint search rule and the fit-file format the solver reads back."""
import json

import numpy as np
import pytest

from ae_amd.optimizer import GPUFusedMoEModel, PiecewiseLinearFitter


def _profile(n, y):
    return [{"input_params": {"num_tokens": int(a)}, "latency": float(b)} for a, b in zip(n, y)]


def test_recovers_exact_piecewise_line():
    n = np.array([1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024])
    y = np.where(n <= 64, 2e-6 * n + 4e-4, 5e-6 * n + 2e-4)
    m = GPUFusedMoEModel()
    fit = PiecewiseLinearFitter(min_samples_per_segment=3).fit(m, _profile(n, y))
    p = m.get_parameters()
    assert p["breakpoint"] == 64
    np.testing.assert_allclose([p["a1"], p["b1"], p["a2"], p["b2"]], [2e-6, 4e-4, 5e-6, 2e-4], rtol=1e-9)
    assert fit["best_score"] == pytest.approx(1.0)
    for t, want in zip(n, y):
        assert m.predict(int(t)) == pytest.approx(want, rel=1e-9)


def test_segments_match_scikit_learn_least_squares():
    from sklearn.linear_model import LinearRegression
    rng = np.random.default_rng(0)
    n = np.array([1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256, 384, 512])
    y = np.where(n <= 48, 3e-6 * n + 5e-4, 9e-6 * n + 2e-4) * (1 + 0.03 * rng.standard_normal(n.size))
    m = GPUFusedMoEModel()
    PiecewiseLinearFitter(min_samples_per_segment=3).fit(m, _profile(n, y))
    p = m.get_parameters()
    bp = p["breakpoint"]
    for mask, (a, b) in (((n <= bp), (p["a1"], p["b1"])), ((n > bp), (p["a2"], p["b2"]))):
        lr = LinearRegression().fit(n[mask].reshape(-1, 1).astype(np.float64), y[mask])
        assert a == pytest.approx(lr.coef_[0], rel=1e-9)
        assert b == pytest.approx(lr.intercept_, rel=1e-9, abs=1e-12)


def test_breakpoint_rule_minimizes_max_relative_error():
    rng = np.random.default_rng(1)
    n = np.arange(1, 41) * 8
    y = np.maximum(4e-4, 1e-6 * n) * (1 + 0.02 * rng.standard_normal(n.size))
    f = PiecewiseLinearFitter(min_samples_per_segment=4)
    m = GPUFusedMoEModel()
    fit = f.fit(m, _profile(n, y))
    cands = f.candidates(n.astype(float))
    assert all(np.sum(n <= c) >= 4 and np.sum(n > c) >= 4 for c in cands)
    scores = {r["breakpoint"]: r["score"] for r in fit["breakpoint_search_results"]}
    assert set(scores) == set(cands)
    assert fit["best_breakpoint"] == max(cands, key=lambda c: (scores[c], -cands.index(c)))
    assert fit["best_score"] == pytest.approx(1 / (1 + fit["training_metrics"]["max_relative_error"]))


def test_predict_semantics_and_fit_file(tmp_path):
    m = GPUFusedMoEModel()
    with pytest.raises(ValueError):
        m.predict(4)
    m.set_parameters({"a1": -1.0, "b1": 1.0, "a2": 2.0, "b2": -3.0, "breakpoint": 2})
    assert m.predict(2) == 0.0  # left segment includes the breakpoint: -2 + 1 -> floored at 0
    assert m.predict(3) == 3.0
    n = np.array([1, 2, 3, 4, 5, 6, 7, 8])
    y = 1e-5 * n + 1e-4
    f = PiecewiseLinearFitter(min_samples_per_segment=3)
    fit = f.fit(m, _profile(n, y))
    ev = f.evaluate_fit(m, _profile(n, y))
    path = f.save_fit_results(m, fit, ev, str(tmp_path / "fit" / "gpu_moe.json"))
    with open(path) as fh:
        data = json.load(fh)
    m2 = GPUFusedMoEModel()
    m2.set_parameters(data["parameters"])  # what the solver does with the file
    assert all(m2.predict(int(t)) == pytest.approx(m.predict(int(t))) for t in n)
