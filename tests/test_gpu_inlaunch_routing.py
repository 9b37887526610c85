"""Routing inside the gate/up launch for small batches (no routing kernel): every entry point
it covers gives the same bits as with the routing kernels, and matches the oracle, through
the C ABI -- routing from logits (fused forward, shared-expert blocks), from caller ids
(stack_fused_moe, dropped and repeated ids included) and from the norm kernel's picks (the
layer call)."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import (fused_down_max_tokens, fused_moe_forward, fused_moe_shared_forward,
                           moe_layer_forward, routing_in_gateup, stack_fused_moe)
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, H, E, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    return x, logits


def _both(fn):
    outs = {}
    for on in (True, False):
        with routing_in_gateup(on):
            outs[on] = fn()
        torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,P", [
    (1, 256, 128, 8, 2, 8),
    (3, 128, 256, 64, 6, 70),      # 18 assignments over 64 experts, some slots unmapped
    (4, 256, 128, 60, 4, 60),
    (16, 256, 128, 8, 2, 8),       # one token tile
    (32, 256, 128, 8, 2, 12),      # 64 assignments, two token tiles
    (8, 128, 128, 16, 8, 16),      # 64 assignments over 16 experts
])
def test_fused_forward_in_launch_routing(dtype, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T * 3 + E)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k)
    if P > E:
        slots[1] = P + 5  # an expert outside the pool: its assignments are dropped
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T", [1, 2, 4])
def test_shared_block_in_launch_routing(T):
    """DeepSeek-V2-Lite block: the shared expert's workgroups start without routing."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=50 + T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=51)
    g = torch.Generator(device=DEV).manual_seed(52)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    outs = _both(lambda: fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page,
                                                  None, 1.0, inplace=False))
    assert torch.equal(outs[True], outs[False])
    y_ref, _, _ = ref.fused_moe_shared_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                               slots.cpu().numpy(), k, False, "bf16",
                                               shared_page=to_oracle(page))
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]


def test_stack_fused_moe_in_launch_routing_caller_ids():
    T, H, I, E, k = 6, 256, 128, 8, 3
    x, _ = _inputs(T, H, E, torch.bfloat16, seed=61)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=62)
    slots[5] = 1000
    ids = torch.tensor([[0, 9, 5], [2, 2, 7], [-1, 5, 8], [3, 1, 0], [7, 6, 4], [1, 1, 1]],
                       dtype=torch.int32, device=DEV)
    w = torch.rand((T, k), generator=torch.Generator(device=DEV).manual_seed(63), device=DEV)
    logits = torch.zeros((T, E), dtype=torch.bfloat16, device=DEV)
    outs = _both(lambda: stack_fused_moe(x.clone(), pool, slots, logits, w, ids, False))
    assert torch.equal(outs[True], outs[False])
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("T,E,k", [(2, 8, 2), (8, 64, 6), (32, 8, 2)])
def test_layer_call_in_launch_routing(T, E, k):
    """The layer call from two tokens up: the norm kernel's picks sorted inside gate/up."""
    H, I, dt = 256, 256, torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(70 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(dt)
    r = torch.randn((T, H), generator=g, device=DEV).to(dt)
    nw = (torch.randn((H,), generator=g, device=DEV) * 0.1 + 1).to(dt)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(dt)
    pool, slots = make_pool(E, H, I, dt, num_slots=E + 3, seed=71)

    def run():
        xx, rr = x.clone(), r.clone()
        y, (lg, w, ids) = moe_layer_forward(xx, rr, nw, 1e-6, gw, pool, slots, k, E <= 8,
                                            return_routing=True)
        return y, rr, lg, w, ids

    outs = _both(run)
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,P", [
    (8, 256, 128, 64, 6, 70),      # 48 assignments in 8 top-k passes: the multi-wave form
    (20, 128, 128, 64, 6, 64),     # 120 assignments, two token tiles
    (40, 256, 128, 60, 4, 60),     # 160 assignments, three token tiles
    (64, 128, 128, 8, 4, 10),      # 256 assignments, four token tiles
    (50, 256, 256, 16, 5, 20),
])
def test_fused_forward_in_launch_routing_multi_wave(dtype, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T * 5 + E)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k + 1)
    if P > E:
        slots[2] = P + 9
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T", [16, 32, 42])
def test_deepseek_block_in_launch_routing_multi_wave(T):
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=90 + T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=91)
    g = torch.Generator(device=DEV).manual_seed(92)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    outs = _both(lambda: fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page,
                                                  None, 1.0, inplace=False))
    assert torch.equal(outs[True], outs[False])


@pytest.mark.parametrize("T,E,k", [(16, 64, 6), (40, 60, 4)])
def test_layer_call_in_launch_routing_multi_wave(T, E, k):
    H, I, dt = 256, 128, torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(95 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(dt)
    r = torch.randn((T, H), generator=g, device=DEV).to(dt)
    nw = (torch.randn((H,), generator=g, device=DEV) * 0.1 + 1).to(dt)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(dt)
    pool, slots = make_pool(E, H, I, dt, num_slots=E + 3, seed=96)

    def run():
        xx, rr = x.clone(), r.clone()
        y, (lg, w, ids) = moe_layer_forward(xx, rr, nw, 1e-6, gw, pool, slots, k, False,
                                            return_routing=True)
        return y, rr, lg, w, ids

    outs = _both(run)
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,H,I,E,k,P,logits_dt", [
    (16, 256, 128, 64, 6, 70, torch.bfloat16),   # 16 tokens x 64 lanes: top-k in its own launch
    (42, 128, 128, 64, 6, 64, torch.bfloat16),   # 252 assignments, three token tiles
    (24, 256, 128, 32, 8, 40, torch.bfloat16),
    (4, 256, 128, 8, 2, 8, torch.float32),       # logits in another dtype than the activations
    (40, 128, 256, 60, 4, 60, torch.float32),
])
def test_fused_forward_topk_launch_sort_in_gateup(T, H, I, E, k, P, logits_dt):
    """A top-k too large to repeat in every gate/up workgroup (or logits in another dtype) runs
    as its own launch; the gate/up launch sorts its ids."""
    dtype = torch.bfloat16
    x, _ = _inputs(T, H, E, dtype, seed=T * 11 + E)
    logits = (torch.randn((T, E), generator=torch.Generator(device=DEV).manual_seed(T + 1),
                          device=DEV) * 2.0).to(logits_dt)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k + 2)
    if P > E:
        slots[3] = P + 1
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, "bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


def _stack_all_paths(x, pool, slots, logits, w, ids, fused):
    """stack_fused_moe with routing inside gate/up and with the routing kernels, for a fused-down
    setting (None: the default rule)."""
    with fused_down_max_tokens(fused):
        return _both(lambda: stack_fused_moe(x.clone(), pool, slots, logits, w, ids, False))


@pytest.mark.parametrize("T,k,fused", [
    (16, 2, None),   # expert 0 takes all 32 assignments, span 16: two ranges, split down
    (8, 4, 8),       # 32 assignments on one expert through the fused down + combine
    (8, 4, 0),       # the same on the split down kernel + combine
    (32, 2, None),   # 64 assignments, span 32: two ranges
])
def test_repeated_caller_ids_beyond_one_range(T, k, fused):
    """Caller ids that repeat one expert within every token give that expert more assignments
    than one token range holds: the one-wave routing must emit every range of it."""
    H, I, E = 256, 128, 8
    x, _ = _inputs(T, H, E, torch.bfloat16, seed=200 + T + k)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=201)
    ids = torch.zeros((T, k), dtype=torch.int32, device=DEV)
    w = torch.rand((T, k), generator=torch.Generator(device=DEV).manual_seed(202), device=DEV)
    logits = torch.zeros((T, E), dtype=torch.bfloat16, device=DEV)
    outs = _stack_all_paths(x, pool, slots, logits, w, ids, fused)
    assert torch.equal(outs[True], outs[False])
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]


def test_repeated_caller_ids_more_ranges_than_experts():
    """64 experts, 16 tokens of top-8: tokens 0-7 cover every expert once, tokens 8-15 pick
    expert 0 eight times each. Expert 0 then holds 65 assignments (5 ranges of 16), 68 ranges in
    all -- more than one per expert, in the gate/up launch's multi-wave form."""
    T, H, I, E, k = 16, 128, 128, 64, 8
    x, _ = _inputs(T, H, E, torch.bfloat16, seed=210)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=211)
    ids = torch.zeros((T, k), dtype=torch.int32)
    ids[:8] = torch.arange(64, dtype=torch.int32).view(8, 8)
    ids = ids.to(DEV)
    w = torch.rand((T, k), generator=torch.Generator(device=DEV).manual_seed(212), device=DEV)
    logits = torch.zeros((T, E), dtype=torch.bfloat16, device=DEV)
    outs = _stack_all_paths(x, pool, slots, logits, w, ids, None)
    assert torch.equal(outs[True], outs[False])
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]


# Many one-range experts with at least 8 items per range (the routing kernels' records then
# put the expert launches' items in XCD order; inside the gate/up launch the plain order stays):
# the one-wave form (4 tokens of top-16), the multi-wave form from logits (8 tokens of top-6), its
# caller-ids form through the top-k launch (16 tokens of top-6: the own-range routing of the
# non-writer workgroups), and a grid that walks several items per workgroup (ffn 2048: 32 items
# per range). Same bits as with the routing kernels, and the oracle.
@pytest.mark.parametrize("T,H,I,E,k", [
    (4, 256, 512, 64, 16),
    (8, 256, 512, 64, 6),
    (16, 256, 512, 64, 6),
    (8, 256, 2048, 64, 6),
])
def test_in_launch_routing_many_experts(T, H, I, E, k):
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=T * 7 + I + k)
    pool, slots = make_pool(E, H, I, dtype, seed=E + I + k)
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T,H,I,E,k,P", [
    (43, 256, 128, 64, 6, 70),     # 258 assignments: past the routing kernel's one-wave sort
    (64, 128, 256, 64, 6, 64),     # 384
    (64, 256, 128, 32, 8, 36),     # 512, the largest sort inside gate/up
    (57, 128, 128, 60, 7, 60),     # 399, ragged token tiles
])
def test_fused_forward_sort_in_gateup_past_256(T, H, I, E, k, P):
    """257..512 assignments: the top-k launch, then the gate/up launch sorts its ids (one wave
    in the records' writer, the own range in every other workgroup) -- the routing kernels'
    records and outputs, bit for bit, and the oracle's."""
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=T * 13 + E)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k + 3)
    if P > E:
        slots[4] = P + 2
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, "bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T", [48, 64])
def test_deepseek_block_sort_in_gateup_past_256(T):
    """The DeepSeek-V2-Lite block at 48 and 64 tokens (288 and 384 assignments)."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=110 + T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=111)
    g = torch.Generator(device=DEV).manual_seed(112)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    outs = _both(lambda: fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page,
                                                  None, 1.0, inplace=False, return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y_ref, _, _ = ref.fused_moe_shared_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                               slots.cpu().numpy(), k, False, "bf16",
                                               shared_page=to_oracle(page))
    assert max_rel_err(f32_of(outs[True][0]), y_ref) <= TOL[torch.bfloat16]


def test_stack_and_layer_call_sort_in_gateup_past_256():
    """Caller ids (repeated, dropped, out of range) at 400 assignments through stack_fused_moe,
    and the layer call's norm picks at 384."""
    T, H, I, E, k = 50, 256, 128, 64, 8
    x, _ = _inputs(T, H, E, torch.bfloat16, seed=121)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=122)
    slots[9] = 1000
    g = torch.Generator(device=DEV).manual_seed(123)
    ids = torch.randint(0, E, (T, k), generator=g, device=DEV, dtype=torch.int32)
    ids[0, :3] = 5
    ids[1, 2] = -1
    ids[2, 4] = E + 3
    w = torch.rand((T, k), generator=g, device=DEV)
    logits = torch.zeros((T, E), dtype=torch.bfloat16, device=DEV)
    outs = _both(lambda: stack_fused_moe(x.clone(), pool, slots, logits, w, ids, False))
    assert torch.equal(outs[True], outs[False])
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]

    T, E, k, dt = 64, 64, 6, torch.bfloat16
    x = torch.randn((T, H), generator=g, device=DEV).to(dt)
    r = torch.randn((T, H), generator=g, device=DEV).to(dt)
    nw = (torch.randn((H,), generator=g, device=DEV) * 0.1 + 1).to(dt)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(dt)
    pool, slots = make_pool(E, H, I, dt, num_slots=E + 3, seed=124)

    def run():
        xx, rr = x.clone(), r.clone()
        y, (lg, w, ids) = moe_layer_forward(xx, rr, nw, 1e-6, gw, pool, slots, k, False,
                                            return_routing=True)
        return y, rr, lg, w, ids

    outs = _both(run)
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,H,I,E,k,P,hot", [
    (96, 256, 128, 64, 6, 70, 0),      # 576 assignments, T > span: several ranges per expert possible
    (128, 128, 256, 64, 6, 64, 0),     # 768, the largest sort inside gate/up
    (128, 256, 256, 8, 2, 8, 2),       # experts over 64 tokens: two to four ranges each
    (200, 128, 128, 16, 3, 18, 3),     # 600, three experts with hot logits
])
def test_fused_forward_sort_in_gateup_several_ranges(T, H, I, E, k, P, hot):
    """Given ids (the top-k launch's) past one token range per expert: the gate/up launch sorts
    them (records of several ranges per expert, weights read side by side with normal caching),
    with the routing kernels' records and outputs bit for bit, and the oracle's."""
    dtype = torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(T + E + k)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    lg = torch.randn((T, E), generator=g, device=DEV) * 2.0
    lg[:, :hot] += 4.0  # most tokens pick the first `hot` experts
    logits = lg.to(dtype)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + k + 5)
    if P > E:
        slots[E - 1] = P + 4
    outs = _both(lambda: fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y, w, ids = outs[True]
    if hot:
        assert int((ids == 0).sum()) > 64  # expert 0 spans several ranges
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), k, True, "bf16")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T", [96, 128])
def test_deepseek_block_sort_in_gateup_several_ranges(T):
    """The DeepSeek-V2-Lite block at 96 and 128 tokens (576 and 768 assignments)."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=130 + T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=131)
    g = torch.Generator(device=DEV).manual_seed(132)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    outs = _both(lambda: fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page,
                                                  None, 1.0, inplace=False, return_routing=True))
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
    y_ref, _, _ = ref.fused_moe_shared_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                               slots.cpu().numpy(), k, False, "bf16",
                                               shared_page=to_oracle(page))
    assert max_rel_err(f32_of(outs[True][0]), y_ref) <= TOL[torch.bfloat16]


def test_stack_and_layer_call_several_ranges():
    """Caller ids at 700 assignments with one expert named by most tokens (several ranges),
    repeats and drops, through stack_fused_moe; the layer call's norm picks at 128 tokens."""
    T, H, I, E, k = 100, 256, 128, 64, 7
    x, _ = _inputs(T, H, E, torch.bfloat16, seed=141)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=142)
    slots[9] = 1000
    g = torch.Generator(device=DEV).manual_seed(143)
    ids = torch.randint(0, E, (T, k), generator=g, device=DEV, dtype=torch.int32)
    ids[:90, 0] = 3        # expert 3 takes 90+ assignments: two ranges
    ids[0, :3] = 5
    ids[1, 2] = -1
    ids[2, 4] = E + 3
    w = torch.rand((T, k), generator=g, device=DEV)
    logits = torch.zeros((T, E), dtype=torch.bfloat16, device=DEV)
    outs = _both(lambda: stack_fused_moe(x.clone(), pool, slots, logits, w, ids, False))
    assert torch.equal(outs[True], outs[False])
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), "bf16", E)
    assert max_rel_err(f32_of(outs[True]), y_ref) <= TOL[torch.bfloat16]

    T, E, k, dt = 128, 64, 6, torch.bfloat16
    x = torch.randn((T, H), generator=g, device=DEV).to(dt)
    r = torch.randn((T, H), generator=g, device=DEV).to(dt)
    nw = (torch.randn((H,), generator=g, device=DEV) * 0.1 + 1).to(dt)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(dt)
    pool, slots = make_pool(E, H, I, dt, num_slots=E + 3, seed=144)

    def run():
        xx, rr = x.clone(), r.clone()
        y, (lg, w, ids) = moe_layer_forward(xx, rr, nw, 1e-6, gw, pool, slots, k, False,
                                            return_routing=True)
        return y, rr, lg, w, ids

    outs = _both(run)
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)
