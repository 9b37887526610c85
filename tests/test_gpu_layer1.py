"""GPU tests of the single-launch layer (one token: gate/up, down projection and combine in one
launch, layer1.hip), through the C ABI:
  - bit-identical outputs and routing to the two-launch form, and parity with the oracle, at
    the DeepSeek-V2-Lite and Qwen1.5-MoE block shapes and on small shapes in three dtypes, on
    NaN-filled outputs and 0xFF workspaces;
  - consecutive calls on one workspace (each call's wait must not be satisfied by the flags of
    the call before it);
  - the give-up path, forced from the host: the gate/up workgroups do not publish, every down
    workgroup gives up after a short bound, writes NaN and sets the status word, and every
    workgroup ends; the next normal call is correct.
"""
import contextlib

import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd import _lib
from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, nan_buffers, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
DCODE = {torch.float32: _lib.SMX_F32, torch.float16: _lib.SMX_F16, torch.bfloat16: _lib.SMX_BF16}


@contextlib.contextmanager
def single_launch(on):
    L = _lib.lib()
    prev = int(L.smx_single_launch_layer())
    L.smx_set_single_launch_layer(1 if on else 0)
    try:
        yield
    finally:
        L.smx_set_single_launch_layer(prev)


def _case(H, I, E, k, Is, dtype, seed, gated):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((1, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((1, E), generator=g, device=DEV) * 2.0).to(dtype)
    sgate = (torch.randn((1, 1), generator=g, device=DEV) * 2.0).to(dtype) if gated else None
    pool, slots = make_pool(E, H, I, dtype, num_slots=E + 3, seed=seed + 1)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(dtype) if Is else None
    return x, logits, sgate, pool, slots, page


def _call(x, logits, pool, slots, k, renorm, page, sgate, scale):
    H, I = x.shape[1], pool.shape[1] // (3 * x.shape[1])
    E = logits.shape[1]
    Is = page.numel() // (3 * H) if page is not None else 0
    nbytes = _lib.lib().smx_moe_shared_workspace_size(1, H, I, E, k, Is, DCODE[x.dtype])
    out, ws = nan_buffers(x, nbytes)
    y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, renorm, page, sgate, scale,
                                         inplace=False, return_routing=True, out=out, workspace=ws)
    return y, w, ids, ws


CASES = [
    # H, I, E, k, Is, gated, renorm, scale
    (2048, 1408, 64, 6, 2816, False, False, 1.0),   # DeepSeek-V2-Lite block
    (2048, 1408, 60, 4, 5632, True, False, 1.0),    # Qwen1.5-MoE block
    (256, 128, 8, 2, 384, True, True, 1.0),
    (512, 256, 16, 4, 256, False, False, 2.5),
    (256, 256, 8, 2, 0, False, True, 1.0),          # no shared expert
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H,I,E,k,Is,gated,renorm,scale", CASES)
def test_single_launch_equals_two_launches(dtype, H, I, E, k, Is, gated, renorm, scale):
    with single_launch(True):
        plan = _lib.plan_info(1, H, I, E, k, DCODE[dtype], Is)
    if not plan["single_launch"]:
        assert dtype == torch.float32, plan  # only fp32 rows of these blocks exceed its registers
        pytest.skip("fp32 rows too long for the single-launch form's registers (two launches run)")
    x, logits, sgate, pool, slots, page = _case(H, I, E, k, Is, dtype, seed=H + I + Is, gated=gated)
    with single_launch(True):
        y1, w1, ids1, _ = _call(x, logits, pool, slots, k, renorm, page, sgate, scale)
    with single_launch(False):
        y2, w2, ids2, _ = _call(x, logits, pool, slots, k, renorm, page, sgate, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(ids1, ids2) and torch.equal(w1, w2)
    assert torch.equal(y1, y2)
    y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, renorm,
        TORCH_TO_ORACLE[dtype], shared_page=None if page is None else to_oracle(page),
        shared_gate_logits=None if sgate is None else f32_of(sgate), routed_scaling_factor=scale)
    np.testing.assert_array_equal(ids1.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w1.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y1), y_ref, TOL[dtype], case=f"single launch H={H} I={I} E={E} k={k} Is={Is} {dtype}")


def test_routed_only_forward_takes_the_single_launch():
    """smx_fused_moe_forward (no shared expert) at one token, a shape whose down projection
    fuses with the combine."""
    H, I, E, k = 512, 256, 8, 2
    with single_launch(True):
        assert _lib.plan_info(1, H, I, E, k, _lib.SMX_BF16)["single_launch"] == 1
    assert _lib.plan_info(1, H, I, E, k, _lib.SMX_BF16)["single_launch"] == 0  # off by default
    x, logits, _, pool, slots, _ = _case(H, I, E, k, 0, torch.bfloat16, seed=5, gated=False)
    outs = []
    for on in (True, False):
        with single_launch(on):
            outs.append(fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_consecutive_calls_on_one_workspace():
    """Each call's down workgroups wait for their own call's publications: eight calls with
    different inputs on one workspace, each equal to the two-launch result of its inputs."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    _, _, _, pool, slots, page = _case(H, I, E, k, Is, torch.bfloat16, seed=7, gated=False)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(1, H, I, E, k, Is, _lib.SMX_BF16)
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=DEV)
    ys, inputs = [], []
    with single_launch(True):
        for i in range(8):
            g = torch.Generator(device=DEV).manual_seed(100 + i)
            x = torch.randn((1, H), generator=g, device=DEV).to(torch.bfloat16)
            logits = (torch.randn((1, E), generator=g, device=DEV) * 2.0).to(torch.bfloat16)
            inputs.append((x, logits))
            ys.append(fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0,
                                               inplace=False, workspace=ws))
    with single_launch(False):
        for (x, logits), y in zip(inputs, ys):
            want = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0,
                                            inplace=False)
            torch.cuda.synchronize()
            assert torch.equal(y, want)


def test_give_up_path_ends_every_workgroup():
    """Forced from the host: the gate/up workgroups never publish and the bound is 200 us.
    Every down workgroup gives up: every output is NaN and the status word holds the call's
    value; the launch ends normally and the next normal call is correct."""
    H, I, E, k, Is = 256, 128, 8, 2, 384
    x, logits, sgate, pool, slots, page = _case(H, I, E, k, Is, torch.bfloat16, seed=9, gated=True)
    with single_launch(True):
        plan = _lib.plan_info(1, H, I, E, k, _lib.SMX_BF16, Is)
    assert plan["single_launch"] == 1
    status = plan["sync_offset"] + 8 * plan["sync_blocks"]
    nbytes = _lib.lib().smx_moe_shared_workspace_size(1, H, I, E, k, Is, _lib.SMX_BF16)
    ws = torch.zeros((nbytes,), dtype=torch.uint8, device=DEV)
    L = _lib.lib()
    try:
        L.smx_set_layer_sync_test(0, 200)
        with single_launch(True):
            y = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, page, sgate, 1.0,
                                         inplace=False, workspace=ws)
        torch.cuda.synchronize()
    finally:
        L.smx_set_layer_sync_test(1, -1)
    assert torch.isnan(y.float()).all()
    assert int(ws[status:status + 8].cpu().view(torch.int64)[0]) != 0
    with single_launch(True):
        y1 = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, page, sgate, 1.0,
                                      inplace=False, workspace=ws)
    with single_launch(False):
        y2 = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, page, sgate, 1.0,
                                      inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.isfinite(y1.float()).all()


def test_graph_capture_uses_two_launches():
    """Under stream capture the two-launch form is recorded (a graph would replay one call
    value); replays with eager calls between them match the eager result."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x, logits, _, pool, slots, page = _case(H, I, E, k, Is, torch.bfloat16, seed=11, gated=False)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(1, H, I, E, k, Is, _lib.SMX_BF16)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=DEV)
    y = torch.empty_like(x)
    with single_launch(True):
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
            fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0,
                                     inplace=False)  # eager work between replays
            torch.cuda.synchronize()
