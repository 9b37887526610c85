"""A token whose hidden state holds a NaN (the condition the reference's verify loop checks for,
specmoe/backend/eagle_worker.py:1116 `_detect_nan_if_needed`) poisons its own output row only: the
other tokens' outputs are bit-identical to the same call without the NaN, on every kernel path
-- weight streaming with the fused and the split down projection, several token ranges per
expert, the MFMA-tiled kernels (whose clamped rows past a range repeat valid tokens), the
shared-expert block and the whole layer call (whose NaN token routes on NaN logits)."""
import pytest
import torch

from ae_amd.layers import (fused_moe_forward, fused_moe_shared_forward, moe_layer_forward,
                           tiled_min_tokens)
from tests.helpers import make_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _inputs(T, H, E, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(BF)
    return x, logits, g


def _check(y_clean, y_nan, bad):
    others = [t for t in range(y_clean.shape[0]) if t != bad]
    assert torch.equal(y_nan[others], y_clean[others])
    assert torch.isnan(y_nan[bad].float()).any()


@pytest.mark.parametrize("T,tiled", [(1, False), (2, False), (32, False), (300, False), (1024, True)])
def test_nan_token_stays_in_its_row(T, tiled):
    H, I, E, k = 256, 128, 8, 2
    x, logits, _ = _inputs(T, H, E, seed=T)
    pool, slots = make_pool(E, H, I, BF, seed=T + 1)
    bad = T // 2
    xn = x.clone()
    xn[bad, 7] = float("nan")
    with tiled_min_tokens(0 if tiled else None):
        y0 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
        y1 = fused_moe_forward(xn, logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    if T == 1:
        assert torch.isnan(y1.float()).any()
    else:
        _check(y0, y1, bad)


def test_nan_token_shared_block():
    T, H, I, E, k, Is = 40, 256, 128, 16, 4, 256
    x, logits, g = _inputs(T, H, E, seed=5)
    pool, slots = make_pool(E, H, I, BF, seed=6)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(BF)
    sg = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(BF)
    xn = x.clone()
    xn[11, 100] = float("nan")
    y0 = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sg, 1.0, inplace=False)
    y1 = fused_moe_shared_forward(xn, logits, pool, slots, k, False, page, sg, 1.0, inplace=False)
    torch.cuda.synchronize()
    _check(y0, y1, 11)


@pytest.mark.parametrize("T", [3, 24])
def test_nan_token_layer_call(T):
    H, I, E, k = 256, 128, 16, 4
    x, _, g = _inputs(T, H, E, seed=7 + T)
    res = torch.randn((T, H), generator=g, device=DEV).to(BF)
    nw = (1.0 + 0.1 * torch.randn((H,), generator=g, device=DEV)).to(BF)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(BF)
    pool, slots = make_pool(E, H, I, BF, seed=8 + T)
    bad = 1
    outs = []
    for poison in (False, True):
        h, r = x.clone(), res.clone()
        if poison:
            h[bad, 3] = float("nan")
        moe_layer_forward(h, r, nw, 1e-6, gw, pool, slots, k, True)
        outs.append((h, r))
    torch.cuda.synchronize()
    _check(outs[0][0], outs[1][0], bad)
    _check(outs[0][1], outs[1][1], bad)  # the residual sum: only the poisoned row
