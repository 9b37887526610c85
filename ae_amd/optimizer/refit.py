"""Profile the MoE operator on this GPU and fit the solver's GPU MoE model.

    python -m ae_amd.optimizer.refit --out FIT.json [--tokens 1,2,4,...] [--experts 8
        --hidden 4096 --ffn 14336 --topk 2]

Writes the fit file the solver loads (``parameters``: a1, b1, a2, b2, breakpoint; reference
specmoe/optimizer/solver.py:109-165,171-205) with the profile points and fit metrics.
"""
from __future__ import annotations

import argparse
import json

VERIFY_TOKENS = [1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256, 384, 512, 768, 1024]


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", required=True)
    ap.add_argument("--tokens", default=",".join(str(t) for t in VERIFY_TOKENS))
    ap.add_argument("--experts", type=int, default=8)
    ap.add_argument("--hidden", type=int, default=4096)
    ap.add_argument("--ffn", type=int, default=14336)
    ap.add_argument("--topk", type=int, default=2)
    ap.add_argument("--runs", type=int, default=10)
    ap.add_argument("--min-samples", type=int, default=3)
    args = ap.parse_args(argv)

    from .gpu_fused_moe_model import GPUFusedMoEModel
    from .gpu_fused_moe_operator import GPUFusedMoEOperator, run_profile
    from .piecewise_fitter import PiecewiseLinearFitter

    tokens = [int(t) for t in args.tokens.split(",")]
    op = GPUFusedMoEOperator(num_experts=args.experts, hidden_size=args.hidden,
                             expert_size=args.ffn, top_k=args.topk)
    profile = run_profile(op, tokens, num_warmup=2, num_runs=args.runs)
    for p in profile:
        print(json.dumps({"num_tokens": p["input_params"]["num_tokens"],
                          "latency_us": round(p["latency"] * 1e6, 2)}), flush=True)
    model = GPUFusedMoEModel(num_experts=args.experts, hidden_size=args.hidden,
                             expert_size=args.ffn, top_k=args.topk)
    fitter = PiecewiseLinearFitter(min_samples_per_segment=args.min_samples)
    fit = fitter.fit(model, profile)
    ev = fitter.evaluate_fit(model, profile)
    fit["profile"] = profile
    fitter.save_fit_results(model, fit, ev, args.out)
    print(json.dumps({"parameters": model.get_parameters(), "evaluation": ev}), flush=True)


if __name__ == "__main__":
    main()
