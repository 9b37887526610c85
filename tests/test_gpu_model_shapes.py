"""Full-size MoE blocks of other architectures than the benchmarked ones, at verify-step token
counts: Mixtral-8x22B (hidden 6144, 8 experts of ffn 16384, top-2), DBRX (hidden 6144, 16
experts of ffn 10752, top-4), Qwen2-57B-A14B (hidden 3584, 64 experts of ffn 2560, top-8, a
gated shared expert of ffn 20480) and DeepSeek-V2 (hidden 5120, 160 experts of ffn 1536,
top-6 group-limited over 8 groups of which 3 stay selectable, 2 shared experts, routed
scaling 16). Routing ids and weight bits equal the oracle's; outputs are within the bf16
tolerance. The pools (up to 7.5 GB) stay on the GPU; the oracle gets the picked experts'
pages only, as a compact pool with its own slot map."""
import numpy as np
import pytest
import torch

from ae_amd.layers import (fused_moe_forward, fused_moe_shared_forward, grouped_topk,
                           stack_fused_moe_shared)
from oracle import moe_ref as ref
from tests.helpers import TOL, f32_of, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16

# name: hidden, ffn, experts, top-k, shared ffn, shared gate, renormalise, routed scale,
# (groups, selectable groups) or None
MODELS = {
    "mixtral-8x22b": (6144, 16384, 8, 2, 0, False, True, 1.0, None),
    "dbrx": (6144, 10752, 16, 4, 0, False, True, 1.0, None),
    "qwen2-57b-a14b": (3584, 2560, 64, 8, 20480, True, False, 1.0, None),
    "deepseek-v2": (5120, 1536, 160, 6, 3072, False, False, 16.0, (8, 3)),
}


@pytest.fixture(scope="module", params=list(MODELS))
def model(request):
    H, I, E, k, Is, gated, renorm, scale, groups = MODELS[request.param]
    g = torch.Generator(device=DEV).manual_seed(len(request.param))
    pool = torch.empty((E + 1, 3 * I * H), dtype=BF, device=DEV)  # one spare slot
    for p in range(E + 1):
        pool[p].normal_(0.0, 0.02, generator=g)
    slots = torch.randperm(E + 1, generator=torch.Generator().manual_seed(E))[:E].to(DEV)
    page = None
    if Is:
        page = torch.empty((3 * Is * H,), dtype=BF, device=DEV).normal_(0.0, 0.02, generator=g)
    yield request.param, pool, slots, page
    del pool
    torch.cuda.empty_cache()


def _compact(pool, slots, ids_ref, E):
    """The picked experts' pages and an expert -> compact slot map (-1 elsewhere)."""
    picked = np.unique(ids_ref)
    picked = picked[(picked >= 0) & (picked < E)]
    compact = to_oracle(pool[slots[torch.from_numpy(picked).to(DEV)]])
    cslots = np.full(E, -1, dtype=np.int64)
    cslots[picked] = np.arange(picked.size)
    return compact, cslots


@pytest.mark.parametrize("T", [1, 8, 64])
def test_full_size_block(model, T):
    name, pool, slots, page = model
    H, I, E, k, Is, gated, renorm, scale, groups = MODELS[name]
    g = torch.Generator(device=DEV).manual_seed(1000 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(BF)
    sgate = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(BF) if gated else None
    if groups is not None:
        w, ids = grouped_topk(logits, k, renorm, groups[0], groups[1])
        y = stack_fused_moe_shared(x.clone(), pool, slots, w, ids, page, None, scale, inplace=False)
        w_ref, ids_ref = ref.grouped_topk(f32_of(logits), k, renorm, groups[0], groups[1])
    elif Is:
        y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, renorm, page, sgate,
                                             scale, inplace=False, return_routing=True)
        w_ref, ids_ref = ref.topk_softmax(f32_of(logits), k, renorm)
    else:
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, renorm, inplace=False,
                                      return_routing=True)
        w_ref, ids_ref = ref.topk_softmax(f32_of(logits), k, renorm)
    torch.cuda.synchronize()
    case = f"{name} T={T}"
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref, err_msg=case)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32), err_msg=case)
    compact, cslots = _compact(pool, slots, ids_ref, E)
    y_ref = ref.stack_fused_moe_shared(
        to_oracle(x), compact, cslots, w_ref, ids_ref, ref.BF16,
        shared_page=None if page is None else to_oracle(page),
        shared_gate_logits=None if sgate is None else f32_of(sgate), routed_scaling_factor=scale)
    parity(f32_of(y), y_ref, TOL[BF], case=case)
