"""GPU parity of the routing entry points against the oracle: bit-exact ids, weights and
permutations (smx_topk_softmax, smx_moe_align_block_size)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import moe_align_block_size, select_experts

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_topk(logits: torch.Tensor, k: int, renorm: bool):
    return ref.topk_softmax(logits.float().cpu().numpy(), k, renorm)


@pytest.mark.parametrize("ldt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (64, 6), (5, 1), (256, 8), (128, 16), (1, 1)])
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
