"""Piecewise-linear fit of latency against token count with an exhaustive breakpoint search.

Reference: specmoe/optimizer/performance_simulator/fitter/piecewise_fitter.py:15-330. For
every candidate breakpoint (each measured token count leaving at least
``min_samples_per_segment`` samples on both sides), an ordinary least-squares line is fit on
each side; the candidate's score is 1 / (1 + the largest relative error over all samples) and
the best score wins (the first, on ties). Lines are fit with numpy's least squares.
"""
from __future__ import annotations

import json
import os
from typing import Any, Dict, List, Tuple

import numpy as np


def _line(x: np.ndarray, y: np.ndarray) -> Tuple[float, float]:
    """Least-squares slope and intercept of y = a*x + b."""
    A = np.column_stack([x.astype(np.float64), np.ones(len(x))])
    (a, b), *_ = np.linalg.lstsq(A, y.astype(np.float64), rcond=None)
    return float(a), float(b)


def _r2(y: np.ndarray, p: np.ndarray) -> float:
    ss_res = float(np.sum((y - p) ** 2))
    ss_tot = float(np.sum((y - y.mean()) ** 2))
    return 1.0 - ss_res / ss_tot if ss_tot > 0 else 1.0


class PiecewiseLinearFitter:
    def __init__(self, min_samples_per_segment: int = 5, breakpoint_search_method: str = "exhaustive",
                 relative_error_weight: float = 0.5, root_path: str = None,
                 output_dir: str = "fit_results"):
        if breakpoint_search_method != "exhaustive":
            raise NotImplementedError("only the exhaustive breakpoint search is provided")
        self.min_samples_per_segment = min_samples_per_segment
        self.breakpoint_search_method = breakpoint_search_method
        self.relative_error_weight = relative_error_weight
        self.root_path = root_path
        self.output_dir = output_dir

    @staticmethod
    def _data(profile_data: List[Dict[str, Any]]) -> Tuple[np.ndarray, np.ndarray]:
        pts = [(d["input_params"]["num_tokens"], d["latency"]) for d in profile_data
               if d.get("latency") is not None]
        pts.sort()
        return np.array([p[0] for p in pts], dtype=np.float64), np.array([p[1] for p in pts], dtype=np.float64)

    def candidates(self, n: np.ndarray) -> List[int]:
        m = self.min_samples_per_segment
        return [int(t) for t in np.unique(n) if np.sum(n <= t) >= m and np.sum(n > t) >= m]

    def _fit_at(self, n: np.ndarray, y: np.ndarray, bp: int) -> Dict[str, Any]:
        left, right = n <= bp, n > bp
        if left.sum() < 2 or right.sum() < 2:
            raise ValueError("too few samples in a segment")
        a1, b1 = _line(n[left], y[left])
        a2, b2 = _line(n[right], y[right])
        pred = np.where(left, a1 * n + b1, a2 * n + b2)
        rel = np.abs((pred - y) / y)
        max_rel = float(rel.max())
        return {
            "parameters": {"a1": a1, "b1": b1, "a2": a2, "b2": b2, "breakpoint": int(bp)},
            "overall_score": 1.0 / (1.0 + max_rel),
            "metrics": {"left_r2": _r2(y[left], pred[left]), "right_r2": _r2(y[right], pred[right]),
                        "left_relative_error": float(rel[left].mean()),
                        "right_relative_error": float(rel[right].mean()),
                        "max_relative_error": max_rel},
        }

    def fit(self, model, profile_data: List[Dict[str, Any]], **kwargs) -> Dict[str, Any]:
        n, y = self._data(profile_data)
        cands = self.candidates(n)
        if not cands:
            raise ValueError("no breakpoint candidate leaves enough samples on both sides")
        best, results = None, []
        for bp in cands:
            r = self._fit_at(n, y, bp)
            results.append({"breakpoint": bp, "score": r["overall_score"], "metrics": r["metrics"]})
            if best is None or r["overall_score"] > best["overall_score"]:
                best = r
        model.set_parameters(best["parameters"])
        return {"best_breakpoint": best["parameters"]["breakpoint"], "best_score": best["overall_score"],
                "parameters": best["parameters"], "training_metrics": best["metrics"],
                "breakpoint_search_results": results, "num_samples": int(len(n)),
                "token_range": [float(n.min()), float(n.max())],
                "search_method": self.breakpoint_search_method}

    def evaluate_fit(self, model, profile_data: List[Dict[str, Any]]) -> Dict[str, Any]:
        n, y = self._data(profile_data)
        pred = np.array([model.predict(int(t)) for t in n])
        rel = np.abs((pred - y) / y)
        return {"r2": _r2(y, pred), "rmse": float(np.sqrt(np.mean((pred - y) ** 2))),
                "max_relative_error": float(rel.max()), "avg_relative_error": float(rel.mean()),
                "breakpoint": model.parameters.get("breakpoint")}

    def save_fit_results(self, model, fit_result: Dict[str, Any], evaluation: Dict[str, Any],
                         filepath: str) -> str:
        """JSON with the model's 'parameters' (the key the solver reads back,
        specmoe/optimizer/solver.py:160-165) plus the fit and evaluation details."""
        d = os.path.dirname(filepath)
        if d:
            os.makedirs(d, exist_ok=True)
        with open(filepath, "w", encoding="utf-8") as f:
            json.dump({"model_name": model.name, "parameters": model.get_parameters(),
                       "fit_result": fit_result, "evaluation": evaluation}, f, indent=2)
        return filepath
