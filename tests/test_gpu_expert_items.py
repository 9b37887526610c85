"""GPU tests of the expert-ordered gate/up items (smx_set_gateup_expert_items): batches routed
inside the gate/up launch by its multi-wave form number their routed work items by expert, so
that each workgroup issues its first item's weight loads before it routes the batch. With them
on (the default) every output, top-k weight and id has the bits it has with items numbered by
the routing's ranges, through the C ABI, and the oracle's results:
  - shared-expert blocks and the fused forward from logits (the top-k launch; and the top-k
    inside the gate/up launch with item walks), at the DeepSeek-V2-Lite block shape and on
    small shapes in three dtypes, with experts outside the pool and experts no token picks
    (their logits pushed down: their workgroups' early weight loads are never used);
  - caller ids (stack_fused_moe: repeated, dropped and out-of-range ids) and the layer call
    (the norm kernel's picks);
  - NaN-filled outputs and 0xFF workspaces, and ten calls in a row on one workspace.
"""
import contextlib

import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd import _lib
from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward, moe_layer_forward, stack_fused_moe
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, nan_buffers, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
DCODE = {torch.float32: _lib.SMX_F32, torch.float16: _lib.SMX_F16, torch.bfloat16: _lib.SMX_BF16}
MODES = (0, 1)


@contextlib.contextmanager
def expert_items(on):
    L = _lib.lib()
    prev = int(L.smx_gateup_expert_items())
    assert L.smx_set_gateup_expert_items(on) == 0
    try:
        yield
    finally:
        L.smx_set_gateup_expert_items(prev)


def _inputs(T, H, E, Is, dtype, seed, idle=()):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = torch.randn((T, E), generator=g, device=DEV) * 2.0
    logits[:, list(idle)] = -30.0  # experts no token picks
    logits = logits.to(dtype)
    sgate = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(dtype)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(dtype) if Is else None
    return x, logits, sgate, page


def _block(x, logits, pool, slots, k, renorm, page, sgate, scale):
    T, H = x.shape
    I = pool.shape[1] // (3 * H)
    Is = page.numel() // (3 * H) if page is not None else 0
    nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, logits.shape[1], k, Is, DCODE[x.dtype])
    out, ws = nan_buffers(x, nbytes)
    return fused_moe_shared_forward(x.clone(), logits, pool, slots, k, renorm, page, sgate, scale,
                                    inplace=False, return_routing=True, out=out, workspace=ws)


BLOCKS = [
    # T, H, I, E, k, Is, gated, renorm, scale, num_slots (> E: expert 1 outside the pool), idle
    (32, 2048, 1408, 64, 6, 2816, False, False, 1.0, 64, ()),        # DeepSeek-V2-Lite block
    (32, 2048, 1408, 64, 6, 2816, True, True, 2.5, 66, (0, 9, 63)),
    (32, 256, 128, 64, 6, 384, False, True, 1.0, 70, (5,)),
    (17, 512, 256, 16, 4, 0, False, True, 1.0, 18, ()),    # 68 assignments, top-k in the launch
    (32, 512, 256, 16, 4, 256, True, True, 1.0, 16, (2,)),  # item walk, top-k in the launch
    (30, 256, 384, 32, 6, 0, False, False, 1.0, 33, ()),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,Is,gated,renorm,scale,P,idle", BLOCKS)
def test_expert_items_equal_range_items(dtype, T, H, I, E, k, Is, gated, renorm, scale, P, idle):
    with expert_items(1):
        plan = _lib.plan_info(T, H, I, E, k, DCODE[dtype], Is)
    assert plan["expert_items"] == 1 and not plan["tiled"], plan
    x, logits, sgate, page = _inputs(T, H, E, Is, dtype, seed=T * 5 + E + Is, idle=idle)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + T)
    if P > E:
        slots[1] = P + 5  # outside the pool: expert 1's assignments are dropped
    sg = sgate if gated else None
    outs = {}
    for mode in MODES:
        with expert_items(mode):
            outs[mode] = _block(x, logits, pool, slots, k, renorm, page, sg, scale)
        torch.cuda.synchronize()
    y0, w0, ids0 = outs[0]
    assert torch.isfinite(y0.float()).all()
    y, w, ids = outs[1]
    assert torch.equal(ids, ids0) and torch.equal(w, w0)
    assert torch.equal(y, y0)
    assert not any(bool((ids0 == e).any()) for e in idle)
    if dtype != torch.float32:
        y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
            to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, renorm,
            TORCH_TO_ORACLE[dtype], shared_page=None if page is None else to_oracle(page),
            shared_gate_logits=None if sg is None else f32_of(sg), routed_scaling_factor=scale)
        np.testing.assert_array_equal(ids0.cpu().numpy(), ids_ref)
        np.testing.assert_array_equal(w0.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
        parity(f32_of(outs[1][0]), y_ref, TOL[dtype], case=f"expert items T={T} H={H} E={E} k={k} Is={Is}")


def test_plan_rule():
    """Expert order where under 1 in 20 experts are expected idle and every expert's tokens are
    one pass of at most two tiles: the DeepSeek-V2-Lite block at 32 tokens, not at 16 or 64
    tokens nor the Qwen1.5-MoE block at 32 (11% idle expected); never with the setting off."""
    ds = (2048, 1408, 64, 6, _lib.SMX_BF16, 2816)
    qw = (2048, 1408, 60, 4, _lib.SMX_BF16, 5632)
    assert _lib.plan_info(32, *ds)["expert_items"] == 1
    assert _lib.plan_info(16, *ds)["expert_items"] == 0
    assert _lib.plan_info(64, *ds)["expert_items"] == 0
    assert _lib.plan_info(32, *qw)["expert_items"] == 0
    with expert_items(0):
        assert _lib.plan_info(32, *ds)["expert_items"] == 0


def test_forward_without_shared_expert():
    """smx_fused_moe_forward (no block terms) with experts that get no tokens."""
    T, H, I, E, k = 32, 512, 256, 64, 6
    x, logits, _, _ = _inputs(T, H, E, 0, torch.bfloat16, seed=11, idle=(1, 2, 40))
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=12)
    outs = {}
    for mode in MODES:
        with expert_items(mode):
            outs[mode] = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                           return_routing=True)
        torch.cuda.synchronize()
    for a, b in zip(outs[1], outs[0]):
        assert torch.equal(a, b)
    assert len(torch.unique(outs[0][2])) <= E - 3
    y_ref, _, _ = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                        slots.cpu().numpy(), k, True, ref.BF16)
    parity(f32_of(outs[1][0]), y_ref, TOL[torch.bfloat16], case="expert items, forward")


def test_caller_ids_repeated_dropped_out_of_range():
    """stack_fused_moe routes caller ids in the gate/up launch: a token that names one expert
    twice, ids outside [0, E) and an expert outside the pool."""
    T, H, I, E, k = 32, 512, 256, 64, 6
    x, logits, _, _ = _inputs(T, H, E, 0, torch.bfloat16, seed=13)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=14)
    slots[7] = E + 3
    w, ids = ref.topk_softmax(f32_of(logits), k, False)
    ids = ids.copy()
    ids[0, 1] = ids[0, 0]  # repeated
    ids[3, 2] = -1         # out of range
    ids[5, 4] = E + 2      # out of range
    w_t, ids_t = torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    with expert_items(1):
        assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)["expert_items"] == 1
    outs = {}
    for mode in MODES:
        with expert_items(mode):
            outs[mode] = stack_fused_moe(x.clone(), pool, slots, logits, w_t, ids_t, False)
        torch.cuda.synchronize()
    assert torch.equal(outs[1], outs[0])


def test_layer_call_norm_picks():
    """The layer call at 32 tokens: the norm kernel's picks, sorted in the gate/up launch."""
    T, H, I, E, k, Is = 32, 2048, 1408, 64, 6, 2816
    g = torch.Generator(device=DEV).manual_seed(15)
    hidden = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    residual = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    norm_w = (1.0 + 0.1 * torch.randn((H,), generator=g, device=DEV)).to(torch.bfloat16)
    gate_w = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=16)
    outs = {}
    for mode in MODES:
        with expert_items(mode):
            h, r = hidden.clone(), residual.clone()
            moe_layer_forward(h, r, norm_w, 1e-6, gate_w, pool, slots, k, False, shared_w=page)
            outs[mode] = (h, r)
        torch.cuda.synchronize()
    assert torch.equal(outs[1][0], outs[0][0]) and torch.equal(outs[1][1], outs[0][1])


def test_repeated_calls_on_one_workspace():
    """Ten calls on one 0xFF-filled workspace: identical bits to a fresh workspace."""
    T, H, I, E, k, Is = 32, 2048, 1408, 64, 6, 2816
    x, logits, sgate, page = _inputs(T, H, E, Is, torch.bfloat16, seed=17, idle=(7,))
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=18)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, E, k, Is, _lib.SMX_BF16)
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=DEV)
    with expert_items(0):
        want = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sgate, 1.0,
                                        inplace=False)
    with expert_items(1):
        ys = [fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sgate, 1.0,
                                       inplace=False, workspace=ws) for _ in range(10)]
    torch.cuda.synchronize()
    assert all(torch.equal(y, want) for y in ys)


def test_graph_replays_match_eager():
    """A captured call with expert-ordered items (the top-k launch, then the gate/up launch that
    sorts its ids) replays to the eager result, with eager calls between the replays."""
    T, H, I, E, k, Is = 32, 2048, 1408, 64, 6, 2816
    assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16, Is)["expert_items"] == 1
    x, logits, _, page = _inputs(T, H, E, Is, torch.bfloat16, seed=19, idle=(11,))
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=20)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, E, k, Is, _lib.SMX_BF16)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=DEV)
    y = torch.empty_like(x)
    want = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0, inplace=False)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_moe_shared_forward(x, logits, pool, slots, k, False, page, None, 1.0, inplace=False,
                                 out=y, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused_moe_shared_forward(x, logits, pool, slots, k, False, page, None, 1.0, inplace=False,
                                 out=y, workspace=ws)
    for _ in range(4):
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)
        fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0, inplace=False)
        torch.cuda.synchronize()
