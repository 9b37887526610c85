"""GPU parity of the routing entry points against the oracle: bit-exact ids, weights and
permutations (smx_topk_softmax, smx_moe_align_block_size)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import fused_moe_forward, moe_align_block_size, select_experts
from tests.helpers import TOL, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_topk(logits: torch.Tensor, k: int, renorm: bool):
    return ref.topk_softmax(logits.float().cpu().numpy(), k, renorm)


@pytest.mark.parametrize("ldt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (64, 6), (5, 1), (256, 8), (128, 16), (1, 1),
                                 (12, 3), (17, 4), (33, 6), (40, 8), (9, 9)])
@pytest.mark.parametrize("T", [1, 7, 64, 1000])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_softmax_bit_exact(ldt, E, k, T, renorm):
    g = torch.Generator(device=DEV).manual_seed(T * 1000 + E * 10 + k)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(ldt)
    w, ids = select_experts(torch.empty((T, 16), device=DEV), logits, k, False, renorm)
    torch.cuda.synchronize()
    w_ref, ids_ref = _oracle_topk(logits, k, renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))


def test_topk_softmax_ties():
    x = torch.zeros((4, 8), device=DEV)
    x[1, [2, 5, 6]] = 1.0
    x[2] = torch.tensor([0, 3, 3, 1, 3, 0, 0, 1], dtype=torch.float32)
    x[3] = -1e30  # huge negative: all exps but the max underflow to zero
    x[3, 4] = 0.0
    w, ids = select_experts(x, x, 3, False, False)
    w_ref, ids_ref = _oracle_topk(x, 3, False)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(ids.cpu().numpy()[:3], [[0, 1, 2], [2, 5, 6], [1, 2, 4]])
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))


# The top-k inside the single routing workgroup (fused with the expert sort) or in the top-k
# kernel first: 8 < E <= 64 fuses while T*k <= 512 in one pass of the workgroup's 16 waves (E =
# 64: 128 tokens a pass; E = 12: 512), other E while T*E <= 1024.
@pytest.mark.parametrize("T,E,k", [(48, 64, 6), (85, 64, 6), (86, 64, 6), (128, 64, 6),
                                   (64, 40, 8), (65, 40, 8), (170, 12, 3), (171, 12, 3),
                                   (512, 12, 1), (513, 12, 1), (128, 8, 2), (129, 8, 2),
                                   (10, 100, 4), (11, 100, 4)])
def test_fused_forward_routing_bit_exact(T, E, k):
    H, I = 128, 128
    g = torch.Generator(device=DEV).manual_seed(7 * T + E)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=E + 1)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                  return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, "bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("E,k", [(64, 6), (12, 3)])
def test_nan_logits_same_picks_on_every_path(E, k):
    """A token with a NaN logit has NaN probabilities: every path ranks them below every number
    and picks the lowest expert indices, with NaN weights (the oracle's argmax would differ, so
    the paths are compared with each other: the top-k kernel, the one-wave routing of one
    token, and the routing workgroup's top-k)."""
    H, I = 128, 128
    base = torch.randn((64, E), generator=torch.Generator(device=DEV).manual_seed(5), device=DEV)
    base[3, 1] = float("nan")
    base[40, E - 1] = float("nan")
    logits = base.to(torch.bfloat16)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=9)
    w_k, ids_k = select_experts(logits, logits, k, False, False)
    for t in (3, 40):
        assert ids_k[t].tolist() == list(range(k))
        assert torch.isnan(w_k[t]).all()
    x = torch.randn((64, H), device=DEV).to(torch.bfloat16)
    _, w_f, ids_f = fused_moe_forward(x.clone(), logits, pool, slots, k, False, inplace=False,
                                      return_routing=True)
    _, w_1, ids_1 = fused_moe_forward(x[3:4].clone(), logits[3:4], pool, slots, k, False,
                                      inplace=False, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(ids_f, ids_k) and torch.equal(ids_1, ids_k[3:4])
    assert torch.equal(torch.isnan(w_f), torch.isnan(w_k))
    ok = ~torch.isnan(w_k)
    assert torch.equal(w_f[ok], w_k[ok])
    assert torch.isnan(w_1).all()


def test_topk_softmax_empty():
    x = torch.empty((0, 8), device=DEV)
    w, ids = select_experts(x, x, 2, False, True)
    assert w.shape == (0, 2) and ids.shape == (0, 2)


def _check_align(ids: torch.Tensor, bm: int, E: int):
    s, e, n = moe_align_block_size(ids, bm, E)
    torch.cuda.synchronize()
    s_ref, e_ref, n_ref = ref.moe_align_block_size(ids.cpu().numpy(), bm, E)
    assert int(n.item()) == int(n_ref[0])
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(e.cpu().numpy(), e_ref)


def test_align_docstring_example():
    path = os.path.join(os.path.dirname(__file__), "golden", "align_docstring_kat.json")
    with open(path) as f:
        kat = json.load(f)
    ids = torch.tensor(kat["topk_ids"], dtype=torch.int32, device=DEV)
    s, e, n = moe_align_block_size(ids, kat["block_size"], kat["num_experts"])
    ntp = kat["num_tokens_post_pad"]
    assert int(n.item()) == ntp
    assert s.cpu().tolist()[:ntp] == kat["sorted_token_ids"]
    assert e.cpu().tolist()[:ntp // kat["block_size"]] == kat["expert_ids"]
    _check_align(ids, kat["block_size"], kat["num_experts"])


@pytest.mark.parametrize("T,E,k,bm", [(32, 8, 2, 16), (64, 8, 2, 64), (1, 8, 2, 16), (64, 60, 4, 16),
                                      (128, 64, 6, 64), (4096, 8, 2, 64), (8192, 2, 2, 16),
                                      (3000, 256, 5, 7), (100, 1, 1, 1)])
def test_align_random(T, E, k, bm):
    g = torch.Generator().manual_seed(T + E + k + bm)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    _check_align(ids.to(DEV), bm, E)


def test_align_skewed_and_edge_cases():
    # every assignment on one expert
    _check_align(torch.full((50, 1), 3, dtype=torch.int32, device=DEV), 16, 8)
    # empty input
    s, e, n = moe_align_block_size(torch.empty((0, 2), dtype=torch.int32, device=DEV), 16, 8)
    assert int(n.item()) == 0
    assert bool((s == 0).all()) and bool((e == -1).all())
    # maximum supported size
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 64, (2048, 8), generator=g, dtype=torch.int32)
    _check_align(ids.to(DEV), 32, 64)
