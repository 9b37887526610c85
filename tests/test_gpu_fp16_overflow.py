"""fp16 layers whose intermediates overflow: gate/up outputs, the SwiGLU product or the weighted
down outputs beyond 65504 round to +-inf at the same rounding points as the reference's fp16
stores (specmoe/layers/fused_moe_kernel.py:203,337,344-347), and inf - inf in a sum is NaN.
Which outputs are finite, +inf, -inf or NaN does not depend on the summation order, so it must
equal the oracle's exactly; the finite outputs are within the fp16 tolerance. Covers the
streaming kernels (fused and split down projection), the MFMA-tiled kernels and the
shared-expert block."""
import numpy as np
import pytest
import torch

from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward, tiled_min_tokens
from oracle import moe_ref as ref
from tests.helpers import TOL, f32_of, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
F16 = torch.float16


def _classes(a):
    a = np.asarray(a, dtype=np.float64)
    return np.where(np.isnan(a), 3, np.where(np.isposinf(a), 1, np.where(np.isneginf(a), 2, 0)))


def _check(y, y_ref, case):
    c, c_ref = _classes(f32_of(y)), _classes(y_ref)
    assert (c_ref != 0).any(), f"{case}: no output overflowed; the case tests nothing"
    assert (c_ref == 0).any(), f"{case}: every output overflowed"
    np.testing.assert_array_equal(c, c_ref, err_msg=case)
    fin = c_ref == 0
    yf, rf = f32_of(y)[fin].astype(np.float64), y_ref[fin].astype(np.float64)
    assert np.abs(yf - rf).max() <= TOL[F16] * np.abs(rf).max(), case


def _case(T, H, I, E, seed, xscale):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = (torch.randn((T, H), generator=g, device=DEV) * xscale).to(F16)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(F16)
    pool = (torch.randn((E, 3 * I * H), generator=g, device=DEV) * 0.5).to(F16)
    slots = torch.randperm(E, generator=torch.Generator().manual_seed(seed)).to(DEV)
    return x, logits, pool, slots


@pytest.mark.parametrize("T,tiled", [(2, False), (32, False), (1024, True)])
def test_fp16_overflow_classes_match_oracle(T, tiled):
    H, I, E, k = 256, 128, 8, 2
    x, logits, pool, slots = _case(T, H, I, E, seed=T, xscale=16.0)
    with tiled_min_tokens(0 if tiled else None):
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                      return_routing=True)
    torch.cuda.synchronize()
    with np.errstate(over="ignore", invalid="ignore"):  # the overflows are the point
        y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                      slots.cpu().numpy(), k, True, ref.F16)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    _check(y, y_ref, f"fp16 overflow T={T} tiled={tiled}")


def test_fp16_overflow_shared_block():
    T, H, I, E, k, Is = 6, 256, 128, 8, 2, 256
    x, logits, pool, slots = _case(T, H, I, E, seed=77, xscale=16.0)
    g = torch.Generator(device=DEV).manual_seed(78)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.2).to(F16)
    sg = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(F16)
    y = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sg, 1.0,
                                 inplace=False)
    torch.cuda.synchronize()
    with np.errstate(over="ignore", invalid="ignore"):
        y_ref, _, _ = ref.fused_moe_shared_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                   slots.cpu().numpy(), k, False, ref.F16,
                                                   shared_page=to_oracle(page),
                                                   shared_gate_logits=f32_of(sg))
    _check(y, y_ref, "fp16 overflow, shared block")
