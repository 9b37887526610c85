"""Tensor forms the reference's callers may pass (specmoe/layers/FusedMoE.py:508-532,
fused_moe_kernel.py:253-349): the expert -> slot map as int32 or as a strided view, router
logits as a column slice of a wider tensor, hidden states as a row window of a larger buffer
(updated in place, the rows around it untouched), caller ids as int64 and weights in bf16.
Each gives the bits of the canonical form (contiguous int64 map, contiguous logits, int32 ids,
fp32 weights)."""
import pytest
import torch

from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward, stack_fused_moe
from tests.helpers import make_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _case(T, H, I, E, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(BF)
    pool, slots = make_pool(E, H, I, BF, num_slots=E + 2, seed=seed + 1)
    return x, logits, pool, slots


@pytest.mark.parametrize("T", [1, 24, 300])
def test_slot_map_and_logit_forms(T):
    H, I, E, k = 256, 128, 16, 4
    x, logits, pool, slots = _case(T, H, I, E, seed=T)
    want = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    # int32 map; a strided view of the map; logits as columns of a wider tensor
    wide = torch.full((T, E + 5), float("nan"), device=DEV, dtype=BF)
    wide[:, 2:2 + E] = logits
    strided = torch.full((2 * E,), -7, dtype=torch.int64, device=DEV)
    strided[::2] = slots
    forms = [(slots.to(torch.int32), logits), (strided[::2], logits), (slots, wide[:, 2:2 + E])]
    for s, lg in forms:
        got = fused_moe_forward(x.clone(), lg, pool, s, k, True, inplace=False)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_hidden_states_window_in_place():
    """In place on rows [3, 3 + T) of a larger buffer: those rows get the layer's output, the
    rows around them keep their bits."""
    T, H, I, E, k = 20, 256, 128, 8, 2
    x, logits, pool, slots = _case(T, H, I, E, seed=5)
    want = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    big = torch.randn((T + 7, H), device=DEV).to(BF)
    before = big.clone()
    big[3:3 + T] = x
    win = big[3:3 + T]
    out = fused_moe_forward(win, logits, pool, slots, k, True)
    torch.cuda.synchronize()
    assert out.data_ptr() == win.data_ptr()
    assert torch.equal(big[3:3 + T], want)
    assert torch.equal(big[:3], before[:3]) and torch.equal(big[3 + T:], before[3 + T:])


def test_shared_block_window_and_int32_map():
    T, H, I, E, k, Is = 9, 256, 128, 8, 2, 256
    x, logits, pool, slots = _case(T, H, I, E, seed=6)
    page = (torch.randn((3 * Is * H,), device=DEV) * 0.02).to(BF)
    sg = (torch.randn((T, 1), device=DEV) * 2.0).to(BF)
    want = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sg, 1.0,
                                    inplace=False)
    big = torch.zeros((T + 4, H), device=DEV, dtype=BF)
    big[2:2 + T] = x
    got = fused_moe_shared_forward(big[2:2 + T], logits, pool, slots.to(torch.int32), k, False, page,
                                   sg.view(-1), 1.0)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert not big[:2].any() and not big[2 + T:].any()


def test_caller_routing_forms():
    """stack_fused_moe on int64 ids and bf16 weights: the library reads int32 ids and fp32
    weights, so these are the canonical call on ids.int() and weights.float()."""
    T, H, I, E, k = 33, 256, 128, 16, 3
    x, logits, pool, slots = _case(T, H, I, E, seed=7)
    g = torch.Generator(device=DEV).manual_seed(8)
    ids = torch.stack([torch.randperm(E, generator=torch.Generator().manual_seed(t))[:k]
                       for t in range(T)]).to(DEV)
    w = (torch.rand((T, k), generator=g, device=DEV) * 0.9 + 0.1).to(BF)
    want = stack_fused_moe(x.clone(), pool, slots, logits, w.float(), ids.to(torch.int32), False)
    got = stack_fused_moe(x.clone(), pool, slots, logits, w, ids.to(torch.int64), False)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
