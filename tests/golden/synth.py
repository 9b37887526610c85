"""Deterministic synthetic inputs of the full-size layer cases that the oracle fixtures in this
directory pin (generated on the host with numpy's PCG64, so every machine with this image
produces the same bits; the GPU tests upload them, the CPU tests feed them to the oracle).

Each case is one MoE call at a real model shape:

  c1_t32        hidden 1024, ffn 2816, 8 experts, top-2, fp32, 32 tokens (4 sequences x 8
                draft tokens); router logits x Wg^T with Wg ~ N(0, 0.02); expert pages in 16
                pool slots through the map [0, 2, 3, 6, 8, 10, 12, 14], unmapped slots NaN.
  mixtral_t1    Mixtral-8x7B layer (4096 / 14336 / 8 experts / top-2), bf16, one verify token,
                Zipf s=1.2 gate bias; logits round(x Wg^T + b).
  dsv2lite_t1   DeepSeek-V2-Lite block (2048 / 64 experts of 1408 / top-6 / shared 2816), bf16,
                one token, logits 2 N(0,1), no renormalisation.
  qwen15_t4     Qwen1.5-MoE-A2.7B block (2048 / 60 experts of 1408 / top-4 / gated shared
                5632), bf16, four tokens, logits 2 N(0,1), shared gate logits N(0,1).

Hidden states are N(0, 1), expert weights N(0, 0.02). Only the pages of experts the routing
picks are filled; every other pool page holds NaN, so a kernel that reads one shows it. A page
depends only on (case seed, expert), not on which other experts are routed.
"""
from __future__ import annotations

import numpy as np

from oracle import moe_ref as ref

CASES = {
    "c1_t32": dict(T=32, H=1024, I=2816, E=8, k=2, dtype=ref.F32, renorm=True, Is=0,
                   gated=False, slots=[0, 2, 3, 6, 8, 10, 12, 14], P=16, logits="gate", seed=0),
    "mixtral_t1": dict(T=1, H=4096, I=14336, E=8, k=2, dtype=ref.BF16, renorm=True, Is=0,
                       gated=False, slots=None, P=8, logits="zipf", seed=1),
    "dsv2lite_t1": dict(T=1, H=2048, I=1408, E=64, k=6, dtype=ref.BF16, renorm=False, Is=2816,
                        gated=False, slots=None, P=64, logits="randn2", seed=2),
    "qwen15_t4": dict(T=4, H=2048, I=1408, E=60, k=4, dtype=ref.BF16, renorm=False, Is=5632,
                      gated=True, slots=None, P=60, logits="randn2", seed=3),
}


def _normal(seed: int, n: int, scale: float) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    a = rng.standard_normal(n, dtype=np.float32)
    if scale != 1.0:
        a *= np.float32(scale)
    return a


def _store(a: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values -> the storage the oracle and the GPU read (bf16 bit patterns)."""
    return ref.f32_to_bf16_bits(a) if dtype == ref.BF16 else np.ascontiguousarray(a, np.float32)


def make_case(name: str) -> dict:
    """The inputs of one case: x, logits (float32 values representable in the logits dtype,
    which is the activation dtype), pool [P, 3*I*H] and slots [E] (int64), the shared page and
    gate logits when the case has them, plus the routing the oracle computes from the logits."""
    c = dict(CASES[name])
    T, H, I, E, k, dt, s = c["T"], c["H"], c["I"], c["E"], c["k"], c["dtype"], c["seed"]
    x = _store(_normal(1000 * s + 1, T * H, 1.0), dt).reshape(T, H)
    xf = ref.to_f32(x, dt)
    if c["logits"] in ("gate", "zipf"):
        wg = ref.to_f32(_store(_normal(1000 * s + 2, E * H, 0.02), dt), dt).reshape(E, H)
        lg = xf @ wg.T
        if c["logits"] == "zipf":
            p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
            lg = lg + ref.round_to(np.log(p / p.sum()).astype(np.float32), dt)
        logits = ref.round_to(lg.astype(np.float32), dt)
    else:
        logits = ref.round_to(_normal(1000 * s + 3, T * E, 2.0).reshape(T, E), dt)
    w, ids = ref.topk_softmax(logits, k, c["renorm"])
    slots = np.asarray(c["slots"] if c["slots"] is not None else range(E), dtype=np.int64)
    nan = np.float32(np.nan)
    pool = np.empty((c["P"], 3 * I * H), dtype=np.uint16 if dt == ref.BF16 else np.float32)
    pool[:] = ref.f32_to_bf16_bits(np.array([nan]))[0] if dt == ref.BF16 else nan
    for e in sorted(set(int(v) for v in ids.reshape(-1))):
        pool[slots[e]] = _store(_normal(1000 * s + 100 + e, 3 * I * H, 0.02), dt)
    out = dict(c, x=x, logits=logits, pool=pool, slot_map=slots, w=w, ids=ids)
    out["shared_page"] = _store(_normal(1000 * s + 4, 3 * c["Is"] * H, 0.02), dt) if c["Is"] else None
    out["shared_gate"] = (ref.round_to(_normal(1000 * s + 5, T, 1.0), dt) if c["gated"] else None)
    return out


def oracle_forward(case: dict):
    """The oracle's (y, w, ids) for a case built by make_case."""
    if case["Is"]:
        return ref.fused_moe_shared_forward(case["x"], case["logits"], case["pool"], case["slot_map"],
                                            case["k"], case["renorm"], case["dtype"],
                                            shared_page=case["shared_page"],
                                            shared_gate_logits=case["shared_gate"])
    return ref.fused_moe_forward(case["x"], case["logits"], case["pool"], case["slot_map"],
                                 case["k"], case["renorm"], case["dtype"])


def bits_of(y: np.ndarray, dtype: str) -> np.ndarray:
    """Output values -> their storage bits (uint16 for bf16, uint32 for fp32)."""
    return ref.f32_to_bf16_bits(y) if dtype == ref.BF16 else np.ascontiguousarray(y, np.float32).view(np.uint32)
