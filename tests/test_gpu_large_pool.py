"""An expert pool larger than 4 GiB whose mapped pages lie past the 4 GiB mark (one straddles
it), every other page NaN: each kernel path reads exactly the mapped pages at their 64-bit
addresses -- the streaming kernels with the split down projection and with the fused down +
combine, the MFMA-tiled kernels, caller routing, the shared-expert block, the single-launch
layer and the whole layer call. The reference's pool (`ws.gpu_cache`, specmoe/layers/
FusedMoE.py:292-338 and the offload engine's cache of `[num_slots, 3*I*H]` pages) is sized
by the cache budget, far beyond 4 GiB for real models. The oracle gets the mapped pages alone,
as a compact pool with the identity map."""
import contextlib

import numpy as np
import pytest
import torch

from ae_amd import _lib
from ae_amd.layers import (fused_moe_forward, fused_moe_shared_forward, moe_layer_forward,
                           stack_fused_moe, tiled_min_tokens)
from oracle import moe_ref as ref
from tests.helpers import TOL, f32_of, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
H, I, E = 256, 256, 8
PAGE = 3 * I * H                                  # elements per page
PAGE_BYTES = PAGE * 2                             # 393216
STRADDLE = (1 << 32) // PAGE_BYTES                # page 10922 spans the 4 GiB mark
SLOTS = [STRADDLE, 11000, 11001, 2, 10950, 5, 11020, STRADDLE + 1]
P = 11024                                         # 4.33 GB of bf16


@pytest.fixture(scope="module")
def big_pool():
    assert STRADDLE * PAGE_BYTES < (1 << 32) < (STRADDLE + 1) * PAGE_BYTES
    pool = torch.full((P, PAGE), float("nan"), dtype=BF, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(41)
    for s in SLOTS:
        pool[s] = (torch.randn((PAGE,), generator=g, device=DEV) * 0.02).to(BF)
    slots = torch.tensor(SLOTS, dtype=torch.int64, device=DEV)
    compact = to_oracle(pool[slots])  # the oracle's pool: mapped pages in expert order
    yield pool, slots, compact
    del pool
    torch.cuda.empty_cache()


@contextlib.contextmanager
def single_launch(on):
    L = _lib.lib()
    prev = int(L.smx_single_launch_layer())
    L.smx_set_single_launch_layer(1 if on else 0)
    try:
        yield
    finally:
        L.smx_set_single_launch_layer(prev)


def _inputs(T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(BF)
    return x, logits


IDENT = np.arange(E, dtype=np.int64)


@pytest.mark.parametrize("T,k,tiled", [(1, 2, False), (4, 2, False), (32, 2, False),
                                       (96, 3, False), (1024, 2, True)])
def test_routed_forward_reads_pages_past_4gib(big_pool, T, k, tiled):
    pool, slots, compact = big_pool
    x, logits = _inputs(T, seed=T + k)
    with tiled_min_tokens(0 if tiled else None):
        plan = _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                      return_routing=True)
    torch.cuda.synchronize()
    assert plan["tiled"] == int(tiled)
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), compact, IDENT, k,
                                                  True, ref.BF16)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y), y_ref, TOL[BF], case=f"pool > 4 GiB T={T} k={k} tiled={tiled}")


def test_caller_routing_reads_pages_past_4gib(big_pool):
    pool, slots, compact = big_pool
    T, k = 16, 3
    x, _ = _inputs(T, seed=77)
    r = np.random.default_rng(77)
    ids = np.stack([r.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = (r.random((T, k)) * 0.9 + 0.1).astype(np.float32)
    logits = torch.zeros((T, E), device=DEV, dtype=BF)
    y = stack_fused_moe(x.clone(), pool, slots, logits, torch.from_numpy(w).to(DEV),
                        torch.from_numpy(ids).to(DEV), False)
    torch.cuda.synchronize()
    y_ref = ref.stack_fused_moe(to_oracle(x), compact, IDENT, w, ids, ref.BF16)
    parity(f32_of(y), y_ref, TOL[BF], case="pool > 4 GiB, caller routing")


@pytest.mark.parametrize("T,single", [(1, False), (1, True), (3, False), (40, False)])
def test_shared_block_reads_pages_past_4gib(big_pool, T, single):
    """The gated shared-expert block; at one token also the single-launch layer."""
    pool, slots, compact = big_pool
    k, Is = 2, 384
    x, logits = _inputs(T, seed=90 + T)
    g = torch.Generator(device=DEV).manual_seed(91 + T)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(BF)
    sgate = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(BF)
    with single_launch(single):
        if single:
            assert _lib.plan_info(1, H, I, E, k, _lib.SMX_BF16, Is)["single_launch"] == 1
        y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, page, sgate,
                                             1.0, inplace=False, return_routing=True)
        torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), compact, IDENT, k, True, ref.BF16, shared_page=to_oracle(page),
        shared_gate_logits=f32_of(sgate))
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y), y_ref, TOL[BF], case=f"pool > 4 GiB shared block T={T} single={single}")


@pytest.mark.parametrize("T", [1, 24])
def test_layer_call_reads_pages_past_4gib(big_pool, T):
    """The whole post-attention call; at one token the norm kernel writes the expert sort."""
    pool, slots, compact = big_pool
    k = 2
    g = torch.Generator(device=DEV).manual_seed(120 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    res = torch.randn((T, H), generator=g, device=DEV).to(BF)
    nw = (1.0 + 0.1 * torch.randn((H,), generator=g, device=DEV)).to(BF)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(BF)
    x0, r0 = x.clone(), res.clone()
    y, (lg, w, ids) = moe_layer_forward(x, res, nw, 1e-6, gw, pool, slots, k, True,
                                        return_routing=True)
    torch.cuda.synchronize()
    y_ref, _, _, w_ref, ids_ref = ref.moe_layer_forward(
        to_oracle(x0), to_oracle(r0), to_oracle(nw), 1e-6, to_oracle(gw), compact, IDENT, k, True,
        ref.BF16, logits=f32_of(lg))
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y), y_ref, TOL[BF], case=f"pool > 4 GiB layer call T={T}")
