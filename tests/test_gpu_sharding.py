"""The sharded forms of the MoE layer, run shard by shard on one GPU through the C ABI: each
shard's output is the partial sum a multi-GPU run would all-reduce, so the shards' outputs
must add up to the unsharded layer (and to the oracle).

Tensor parallel (the reference's scheme, specmoe/layers/FusedMoE.py:301-302,493-505): rank r
holds rows [r*I/n, (r+1)*I/n) of every expert's w1/w3 and those columns of w2, and runs the
full routing. Expert parallel: rank r holds experts [r*E/n, (r+1)*E/n) and maps the others to
no pool slot, so their assignments contribute nothing (the same routing on every rank)."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, H, E, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    return x, logits


def _tp_pool(pool, H, I, n, r):
    """Pages of TP rank r of n: [W1 rows | W3 rows | W2 columns] of its I/n slice."""
    P = pool.shape[0]
    Ip = I // n
    w1 = pool[:, :I * H].view(P, I, H)
    w3 = pool[:, I * H:2 * I * H].view(P, I, H)
    w2 = pool[:, 2 * I * H:].view(P, H, I)
    sl = slice(r * Ip, (r + 1) * Ip)
    return torch.cat([w1[:, sl, :].reshape(P, -1), w3[:, sl, :].reshape(P, -1),
                      w2[:, :, sl].reshape(P, -1)], dim=1).contiguous()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,n", [
    (1, 256, 512, 8, 2, 2),
    (8, 256, 512, 8, 2, 4),
    (32, 512, 1024, 8, 2, 8),     # Mixtral-like routing, TP8 share I/8 = 128
    (64, 256, 1024, 64, 6, 2),
])
def test_tensor_parallel_shards_sum_to_the_layer(dtype, T, H, I, E, k, n):
    x, logits = _inputs(T, H, E, dtype, seed=T + n)
    pool, slots = make_pool(E, H, I, dtype, seed=E + n)
    y_full = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    parts = [fused_moe_forward(x.clone(), logits, _tp_pool(pool, H, I, n, r), slots, k, True,
                               inplace=False) for r in range(n)]
    torch.cuda.synchronize()
    y_sum = sum(f32_of(p) for p in parts)
    y_ref, _, _ = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                        slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    # each shard rounds its own partial once more than the whole layer does
    tol = TOL[dtype] * (2 if dtype != torch.float32 else 1)
    assert max_rel_err(y_sum, f32_of(y_full)) <= tol
    assert max_rel_err(y_sum, y_ref) <= tol


@pytest.mark.parametrize("T,n", [(1, 2), (32, 4), (128, 8)])
def test_expert_parallel_shards_sum_to_the_layer(T, n):
    H, I, E, k, dtype = 256, 512, 16, 2, torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=100 + T)
    pool, slots = make_pool(E, H, I, dtype, seed=101)
    y_full = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    per = E // n
    parts = []
    for r in range(n):
        mine = slots.clone()
        mine[:r * per] = -1
        mine[(r + 1) * per:] = -1
        parts.append(fused_moe_forward(x.clone(), logits, pool, mine, k, True, inplace=False))
    torch.cuda.synchronize()
    y_sum = sum(f32_of(p) for p in parts)
    assert max_rel_err(y_sum, f32_of(y_full)) <= 2 * TOL[dtype]


def test_tensor_parallel_shared_block():
    """DeepSeek-V2-Lite-style block under TP: routed and shared experts both sharded by
    intermediate rows; the shards sum to the block (ungated shared expert, so the block's
    output is linear in the shards' partial outputs up to rounding)."""
    T, H, I, E, k, Is, n = 16, 256, 512, 16, 4, 1024, 2
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=7)
    pool, slots = make_pool(E, H, I, dtype, seed=8)
    g = torch.Generator(device=DEV).manual_seed(9)
    page = (torch.randn((1, 3 * Is * H), generator=g, device=DEV) * 0.02).to(dtype)
    y_full = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page[0], None,
                                      1.0, inplace=False)
    parts = [fused_moe_shared_forward(x.clone(), logits, _tp_pool(pool, H, I, n, r), slots, k,
                                      False, _tp_pool(page, H, Is, n, r)[0], None, 1.0,
                                      inplace=False) for r in range(n)]
    torch.cuda.synchronize()
    y_sum = sum(f32_of(p) for p in parts)
    assert max_rel_err(y_sum, f32_of(y_full)) <= 2 * TOL[dtype]
