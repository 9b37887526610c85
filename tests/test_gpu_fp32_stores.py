"""GPU parity of the opt-in fp16 stores of fp32 runs (the reference's Triton kernel stores an
fp32 run's gate/up and weighted down outputs as fp16, specmoe/layers/fused_moe_kernel.py:
203,248) against the oracle's fp16_outputs mode, on every expert-kernel path, through the C
ABI."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import (fp32_gemm_outputs_fp16, fused_down_max_tokens, fused_moe_forward,
                           tiled_min_tokens)
from tests.helpers import TOL, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"

# the expert-kernel paths: (fused down limit, tiled threshold)
PATHS = {
    "streaming": (0, 1 << 62),
    "fused_down": (8, 1 << 62),
    "tiled": (0, 0),
}


def _inputs(T, H, E, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV)
    logits = torch.randn((T, E), generator=g, device=DEV) * 2.0
    return x, logits


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("T,H,I,E,k", [
    (1, 256, 128, 8, 2),
    (6, 256, 192, 16, 4),
    (32, 1024, 2816, 8, 2),   # the reference's CPU-runnable configuration (fp32)
    (80, 128, 256, 4, 2),
])
def test_fp16_stores_match_oracle(path, T, H, I, E, k):
    fd, tm = PATHS[path]
    if path == "fused_down" and T > 8:
        pytest.skip("the fused down projection takes at most 8 tokens")
    x, logits = _inputs(T, H, E, seed=T + I)
    pool, slots = make_pool(E, H, I, torch.float32, num_slots=E + 1, seed=E)
    with fused_down_max_tokens(fd), tiled_min_tokens(tm):
        with fp32_gemm_outputs_fp16(True):
            y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                          return_routing=True)
        y_plain = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, ref.F32,
                                                  fp16_outputs=True)
    y_true, _, _ = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                         slots.cpu().numpy(), k, True, ref.F32)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    # fp16 rounding of values near a rounding boundary may differ by one fp16 step under a
    # different fp32 accumulation order: the fp16 tolerance
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.float16]
    assert max_rel_err(f32_of(y_plain), y_true) <= TOL[torch.float32]
    assert not torch.equal(y, y_plain)


def test_fp16_stores_leave_bf16_runs_alone():
    T, H, I, E, k = 16, 256, 256, 8, 2
    x, logits = _inputs(T, H, E, seed=5)
    x, logits = x.to(torch.bfloat16), logits.to(torch.bfloat16)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=6)
    y0 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    with fp32_gemm_outputs_fp16(True):
        y1 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
