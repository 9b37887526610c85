"""GPU parity of the tiled expert kernels (MFMA output tiles of 128 tokens, the path for
experts that see many tokens) against the oracle, through the C ABI. Most cases force the
tiled path on small shapes (threshold 0) so the oracle stays fast; the Mixtral cases run it
at its default threshold. Every call runs on an output filled with NaN and a workspace of
0xFF bytes (NaN in every float type): a kernel that reads a row the call did not write, or
LDS a DMA has not filled yet with such a row, turns the output NaN on the first run."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward, tiled_min_tokens
from ae_amd import _lib
from tests.helpers import (TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, nan_buffers,
                           to_oracle, zipf_gate_logits)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, H, E, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    return x, logits


def _oracle_forward(x, logits, pool, slots, k, renorm):
    dt = TORCH_TO_ORACLE[x.dtype]
    return ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                 slots.cpu().numpy(), k, renorm, dt)


def _poisoned(x, logits, pool, k, Is=0):
    """NaN output and 0xFF workspace for a call on these shapes."""
    T, H = x.shape
    E = logits.shape[1]
    I = pool.shape[1] // (3 * H)
    dt = {torch.float32: _lib.SMX_F32, torch.float16: _lib.SMX_F16, torch.bfloat16: _lib.SMX_BF16}[x.dtype]
    if Is:
        nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, E, k, Is, dt)
    else:
        nbytes = _lib.lib().smx_moe_workspace_size(T, H, I, E, k, dt)
    return nan_buffers(x, nbytes)


def _run_and_check(x, logits, pool, slots, k, renorm=True):
    out, ws = _poisoned(x, logits, pool, k)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, renorm, inplace=False,
                                  return_routing=True, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all(), "NaN in the output: a read of unwritten memory"
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    err = max_rel_err(f32_of(y), y_ref)
    assert err <= TOL[x.dtype], err
    return y


CASES = [
    # T, H, I, E, k, slots
    (1, 128, 128, 4, 2, 4),        # one token: every range is ragged
    (16, 128, 128, 4, 2, 6),       # H = 128: two of the four down waves own no rows
    (33, 384, 256, 8, 2, 8),       # H = 384: the second down row group is half owned
    (130, 256, 128, 3, 3, 3),      # every expert sees every token: ranges of 128 + 2
    (300, 128, 256, 4, 2, 6),      # several ranges per expert, ragged last range
    (520, 256, 128, 16, 4, 20),
    (64, 256, 384, 64, 6, 70),     # many experts with few tokens each
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,P", CASES)
def test_tiled_matches_oracle(dtype, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T + H + I)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E)
    with tiled_min_tokens(0):
        _run_and_check(x, logits, pool, slots, k)


@pytest.mark.parametrize("I", [64, 192])
def test_tiled_fp32_partial_column_groups(I):
    """fp32 allows I = 64 or 192: the last gate/up workgroup owns only part of its columns."""
    T, H, E, k = 200, 128, 4, 2
    x, logits = _inputs(T, H, E, torch.float32, seed=I)
    pool, slots = make_pool(E, H, I, torch.float32, seed=I + 1)
    with tiled_min_tokens(0):
        _run_and_check(x, logits, pool, slots, k)


def test_tiled_equals_streaming_within_tolerance_and_is_deterministic():
    T, H, I, E, k = 384, 256, 256, 8, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=5)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=6)
    with tiled_min_tokens(0):
        ys = []
        for _ in range(3):
            out, ws = _poisoned(x, logits, pool, k)
            ys.append(fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                        out=out, workspace=ws))
    with tiled_min_tokens(1 << 62):
        ystream = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    assert all(torch.equal(ys[0], y) for y in ys[1:])
    assert max_rel_err(f32_of(ys[0]), f32_of(ystream)) <= 2 * TOL[torch.bfloat16]


def test_tiled_only_mapped_pages_are_read():
    T, H, I, E, k = 256, 128, 128, 4, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=11)
    pool, _ = make_pool(E, H, I, torch.bfloat16, num_slots=8, seed=12)
    slots = torch.tensor([1, 3, 5, 7], dtype=torch.int64, device=DEV)
    with tiled_min_tokens(0):
        y1 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
        pool[[0, 2, 4, 6]] = float("nan")
        y2 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


SHARED_CASES = [
    # T, H, I, E, k, Is
    (5, 256, 128, 8, 2, 384),
    (130, 128, 256, 6, 3, 256),    # two token ranges of the shared expert
    (300, 256, 128, 8, 2, 640),    # three
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("T,H,I,E,k,Is", SHARED_CASES)
def test_tiled_shared_block_matches_oracle(dtype, gated, T, H, I, E, k, Is):
    g = torch.Generator(device=DEV).manual_seed(T + Is)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    sgate = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(dtype) if gated else None
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(dtype)
    pool, slots = make_pool(E, H, I, dtype, num_slots=E + 2, seed=E + 1)
    scale = 1.0 if gated else 2.5
    with tiled_min_tokens(0):
        out, ws = _poisoned(x, logits, pool, k, Is=Is)  # sized for the plan in force
        y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, gated, page,
                                             sgate, scale, inplace=False, return_routing=True,
                                             out=out, workspace=ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, gated,
        TORCH_TO_ORACLE[dtype], shared_page=to_oracle(page),
        shared_gate_logits=None if sgate is None else f32_of(sgate), routed_scaling_factor=scale)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T,renorm,Is,gated", [(130, True, 0, False), (200, False, 512, True)])
def test_tiled_whole_layer_call(T, renorm, Is, gated):
    """Residual add + RMSNorm + router gate + top-k + MoE in one call, on the tiled kernels."""
    from tests.test_gpu_layer import _layer_case
    with tiled_min_tokens(0):
        _layer_case(T, 256, 256, 8, 2, renorm, Is=Is, gated=gated, seed=T)


@pytest.mark.parametrize("T", [256, 1024])
def test_mixtral_prefill_size_default_threshold(T):
    """Mixtral-8x7B layer at prefill-sized batches: the default threshold picks the tiled
    kernels (expected tokens per expert T*2/8 >= 64)."""
    assert _lib.lib().smx_tiled_min_tokens() == 64
    H, I, E, k = 4096, 14336, 8, 2
    g = torch.Generator(device=DEV).manual_seed(200 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = zipf_gate_logits(x, E, seed=T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=8)
    y = _run_and_check(x, logits, pool, slots, k)
    del pool
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("path", ["tiled", "streaming"])
def test_mixtral_max_assignments_sampled(path):
    """T*top_k = 16384 (the library's limit): Mixtral layer at 8192 tokens on either path.
    Routing is checked bit-exact for every token; outputs against the oracle on a sample of
    tokens (each token's output depends on its own row only)."""
    H, I, E, k, T = 4096, 14336, 8, 2, 8192
    g = torch.Generator(device=DEV).manual_seed(300)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = zipf_gate_logits(x, E, seed=3)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=9)
    with tiled_min_tokens(0 if path == "tiled" else 1 << 62):
        out, ws = _poisoned(x, logits, pool, k)  # sized for the plan in force
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                      return_routing=True, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    w_ref, ids_ref = ref.topk_softmax(f32_of(logits), k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(4))[:24].sort().values
    rows = torch.cat([rows, torch.tensor([0, T - 1])])
    y_ref, _, _ = _oracle_forward(x[rows.to(DEV)], logits[rows.to(DEV)], pool, slots, k, True)
    del pool
    err = max_rel_err(f32_of(y[rows.to(DEV)]), y_ref)
    assert err <= TOL[torch.bfloat16], err
