"""smx_fused_moe_forward_noalloc: the MoE forward with its intermediates in the library's
device-resident scratch instead of a caller workspace. Called through the C ABI and checked
against smx_fused_moe_forward (the same kernels, so the same bits) on two calls in a row, the
second one smaller, and against the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from ae_amd import _lib
from ae_amd.layers._torch import dtype_code, ptr, stream_of, workspace
from oracle import moe_ref as ref
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(entry, x, logits, pool, slots, k, renorm):
    T, H = x.shape
    E = logits.shape[1]
    y = torch.empty_like(x)
    w = torch.empty((T, k), dtype=torch.float32, device=DEV)
    ids = torch.empty((T, k), dtype=torch.int32, device=DEV)
    args = [ptr(x), ptr(y), dtype_code(x.dtype), T, H, ptr(logits), dtype_code(logits.dtype), E, k,
            int(renorm), ptr(pool), pool.shape[0], pool.shape[1], ptr(slots), ptr(w), ptr(ids)]
    if entry == "smx_fused_moe_forward":
        I = pool.shape[1] // (3 * H)
        ws = workspace(_lib.lib().smx_moe_workspace_size(T, H, I, E, k, dtype_code(x.dtype)), x.device)
        args += [ptr(ws), ws.numel()]
    _lib.call(entry, *args, stream_of(x))
    torch.cuda.synchronize()
    return y, w, ids


@pytest.mark.parametrize("dtype,H,I,E,k,P,Ts", [
    (torch.bfloat16, 512, 256, 8, 2, 12, (32, 5)),     # split down + combine, then fused down
    (torch.bfloat16, 256, 128, 64, 6, 64, (40, 3)),    # multi-wave in-launch routing, then one-wave
    (torch.float32, 256, 128, 8, 2, 8, (64, 1)),
])
def test_noalloc_matches_workspace_entry_point(dtype, H, I, E, k, P, Ts):
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E + H)
    for i, T in enumerate(Ts):
        g = torch.Generator(device=DEV).manual_seed(300 + 7 * i + T)
        x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
        logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
        got = _run("smx_fused_moe_forward_noalloc", x, logits, pool, slots, k, True)
        want = _run("smx_fused_moe_forward", x, logits, pool, slots, k, True)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                      slots.cpu().numpy(), k, True, TORCH_TO_ORACLE[dtype])
        np.testing.assert_array_equal(got[2].cpu().numpy(), ids_ref)
        np.testing.assert_array_equal(got[1].cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
        assert max_rel_err(f32_of(got[0]), y_ref) <= TOL[dtype]


def test_noalloc_rejects_sizes_beyond_the_scratch():
    """A batch whose workspace exceeds the scratch is refused before any launch; the output is
    left untouched."""
    H, I, E, k, T = 1024, 2816, 8, 2, 256
    need = _lib.lib().smx_moe_workspace_size(T, H, I, E, k, _lib.SMX_F32)
    assert need > _lib.SMX_NOALLOC_SCRATCH_BYTES
    pool, slots = make_pool(E, H, I, torch.float32, seed=5)
    x = torch.randn((T, H), device=DEV)
    logits = torch.randn((T, E), device=DEV)
    y = torch.full_like(x, 7.0)
    code = _lib.lib().smx_fused_moe_forward_noalloc(
        ptr(x), ptr(y), _lib.SMX_F32, T, H, ptr(logits), _lib.SMX_F32, E, k, 1, ptr(pool),
        pool.shape[0], pool.shape[1], ptr(slots), None, None, stream_of(x))
    assert code == _lib.SMX_ERR_SCRATCH
    assert b"scratch" in _lib.lib().smx_error_string(code)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
