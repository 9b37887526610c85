"""Gate/up grid shapes: waves per workgroup (4, 2, 1) and workgroups walking several items. The
grid changes, the per-wave work and K walk do not, so every forced setting gives the same bits --
routing from logits inside the gate/up launch or from the routing kernels, caller ids,
shared-expert blocks -- and matches the oracle, through the C ABI. The default rule may also
split each item's K walk between wave pairs (rows of at most 16 chunks, at most 32 tokens): a
different fixed summation order, so the default run keeps the routing bits and matches the
oracle, and repeats its own bits."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd import _lib
from ae_amd.layers import (fused_moe_forward, fused_moe_shared_forward, gateup_item_walk,
                           gateup_waves, routing_in_gateup, stack_fused_moe)
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, H, E, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    return x, logits


def _each_waves(fn):
    outs = {}
    for w in (4, 2, 1, None):
        with gateup_waves(w):
            outs[w] = fn()
        torch.cuda.synchronize()
    return outs


def _assert_same(outs, fn=None):
    """Forced settings: the same bits. The default: the same routing bits (the trailing
    outputs), and with `fn` its own bits again on a second call."""
    base = outs[4]
    if fn is not None:
        again = fn()
        for a, b in zip(outs[None], again):
            assert torch.equal(a, b), "default gate/up rule not deterministic"
    for w, o in outs.items():
        if w is None:
            for a, b in zip(base[1:], o[1:]):
                assert torch.equal(a, b), "default gate/up rule changed the routing"
            continue
        for a, b in zip(base, o):
            assert torch.equal(a, b), f"gate/up waves {w} differ from 4"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("in_launch", [True, False])
@pytest.mark.parametrize("T,H,I,E,k,P", [
    (1, 256, 128, 8, 2, 8),
    (1, 256, 384, 64, 6, 64),      # 24 weight tiles per expert over 64 experts
    (3, 128, 256, 64, 6, 70),      # some slots unmapped
    (16, 256, 128, 8, 2, 8),       # one token tile
    (32, 256, 256, 8, 2, 12),      # two token tiles
])
def test_fused_forward_same_bits_every_waves(dtype, in_launch, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T * 5 + I)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k + I)
    if P > E:
        slots[1] = P + 5  # an expert outside the pool: its assignments are dropped
    with routing_in_gateup(in_launch):
        call = lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True,  # noqa: E731
                                         inplace=False, return_routing=True)
        outs = _each_waves(call)
        _assert_same(outs, call)
    y, w, ids = outs[1]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y), y_ref, TOL[dtype], case=f"gate/up waves 1 T={T} I={I} E={E}")
    parity(f32_of(outs[None][0]), y_ref, TOL[dtype], case=f"gate/up default T={T} I={I} E={E}")


@pytest.mark.parametrize("T", [1, 2, 5])
def test_shared_block_same_bits_every_waves(T):
    """DeepSeek-V2-Lite-like block (64 experts, top-6, no renormalisation, a shared expert of
    twice the routed ffn, routed scaling 2.5) at small shapes: the shared expert's workgroups
    follow the waves setting too."""
    H, I, E, k, Is = 256, 128, 64, 6, 384
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=40 + T)
    pool, slots = make_pool(E, H, I, dtype, seed=41)
    g = torch.Generator(device=DEV).manual_seed(42)
    page = (torch.randn(3 * Is * H, generator=g, device=DEV) * 0.02).to(dtype)
    call = lambda: fused_moe_shared_forward(  # noqa: E731
        x.clone(), logits, pool, slots, k, False, page, None, 2.5, inplace=False,
        return_routing=True)
    outs = _each_waves(call)
    _assert_same(outs, call)
    y = outs[1][0]
    y_ref, _, _ = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, False,
        TORCH_TO_ORACLE[dtype], shared_page=to_oracle(page), shared_gate_logits=None,
        routed_scaling_factor=2.5)
    parity(f32_of(y), y_ref, TOL[dtype], case=f"shared block gate/up waves 1 T={T}")
    parity(f32_of(outs[None][0]), y_ref, TOL[dtype], case=f"shared block gate/up default T={T}")


def test_caller_ids_same_bits_every_waves():
    """stack_fused_moe with caller ids, one of them repeated within a token."""
    T, H, I, E, k = 4, 256, 128, 16, 4
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=77)
    pool, slots = make_pool(E, H, I, dtype, seed=78)
    g = torch.Generator(device=DEV).manual_seed(79)
    ids = torch.randint(0, E, (T, k), generator=g, device=DEV, dtype=torch.int32)
    ids[2, 1] = ids[2, 0]
    w = torch.rand((T, k), generator=g, device=DEV, dtype=torch.float32)
    outs = _each_waves(lambda: (stack_fused_moe(x.clone(), pool, slots, logits, w, ids, False),))
    _assert_same(outs)
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    parity(f32_of(outs[1][0]), y_ref, TOL[dtype], case="caller ids gate/up waves 1")
    parity(f32_of(outs[None][0]), y_ref, TOL[dtype], case="caller ids gate/up default")


def _each_walk(fn):
    outs = {}
    for on in (True, False):
        with gateup_item_walk(on):
            outs[on] = fn()
        torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("in_launch", [True, False])
@pytest.mark.parametrize("T,H,I,E,k", [
    (32, 256, 8192, 8, 2),    # ~1000 gate/up items on 512 slots, routing inside the launch
    (64, 256, 4096, 16, 4),   # four token tiles: the top-k launch, the sort in the gate/up launch
    (130, 256, 4096, 8, 2),   # experts over several token ranges (records from the routing kernel)
])
def test_item_walk_same_bits(in_launch, T, H, I, E, k):
    """Gate/up grids larger than one residency: walking several items per workgroup gives the
    same bits as one workgroup per item, and matches the oracle."""
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=T + I)
    pool, slots = make_pool(E, H, I, dtype, seed=E + I)
    with routing_in_gateup(in_launch):
        outs = _each_walk(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True,
                                                    inplace=False, return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    parity(f32_of(y), y_ref, TOL[dtype], case=f"item walk T={T} I={I} E={E}")


def test_item_walk_shared_block_same_bits():
    """DeepSeek-V2-Lite-like block at 32 tokens (shared-expert items first, then routed)."""
    T, H, I, E, k, Is = 32, 256, 1536, 64, 6, 3072
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=91)
    pool, slots = make_pool(E, H, I, dtype, seed=92)
    g = torch.Generator(device=DEV).manual_seed(93)
    page = (torch.randn(3 * Is * H, generator=g, device=DEV) * 0.02).to(dtype)
    outs = _each_walk(lambda: fused_moe_shared_forward(
        x.clone(), logits, pool, slots, k, False, page, None, 1.0, inplace=False,
        return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y_ref, _, _ = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, False,
        TORCH_TO_ORACLE[dtype], shared_page=to_oracle(page), shared_gate_logits=None,
        routed_scaling_factor=1.0)
    parity(f32_of(outs[True][0]), y_ref, TOL[dtype], case="item walk shared block T=32")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("in_launch", [True, False])
@pytest.mark.parametrize("T", [8, 16, 32])
def test_gateup_k_split_shared_block(dtype, in_launch, T):
    """The default rule's K split (wave pairs over the two halves of each item's K walk, summed
    through LDS) on a DeepSeek-V2-Lite-like block it applies to (rows of H 512: 4 chunks in bf16,
    8 in fp32; ffn 1408 and a shared ffn of 2816 give grids of 800+ 4-wave workgroups), against
    the oracle; bit-stable run to run; the forced 4-wave shape (unsplit) against the oracle too."""
    H, I, E, k, Is = 512, 1408, 64, 6, 2816
    dt = {torch.bfloat16: _lib.SMX_BF16, torch.float32: _lib.SMX_F32}[dtype]
    assert _lib.plan_info(T, H, I, E, k, dt, Is)["gateup_ksplit"] == 1, "the default takes the split"
    with gateup_waves(4):
        assert _lib.plan_info(T, H, I, E, k, dt, Is)["gateup_ksplit"] == 0, "a forced shape does not"
    x, logits = _inputs(T, H, E, dtype, seed=300 + T)
    pool, slots = make_pool(E, H, I, dtype, seed=301)
    g = torch.Generator(device=DEV).manual_seed(302)
    page = (torch.randn(3 * Is * H, generator=g, device=DEV) * 0.02).to(dtype)
    call = lambda: fused_moe_shared_forward(  # noqa: E731
        x.clone(), logits, pool, slots, k, False, page, None, 2.5, inplace=False,
        return_routing=True)
    with routing_in_gateup(in_launch):
        outs = _each_waves(call)
        _assert_same(outs, call)
    y_ref, _, _ = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, False,
        TORCH_TO_ORACLE[dtype], shared_page=to_oracle(page), shared_gate_logits=None,
        routed_scaling_factor=2.5)
    parity(f32_of(outs[None][0]), y_ref, TOL[dtype], case=f"K split T={T} {dtype}")
    parity(f32_of(outs[4][0]), y_ref, TOL[dtype], case=f"forced 4 waves T={T} {dtype}")
    if dtype == torch.float32:
        # the split ran: fp32 outputs of another summation order differ in low bits somewhere
        assert not torch.equal(outs[None][0], outs[4][0])
