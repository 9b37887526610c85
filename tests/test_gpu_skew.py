"""Extreme expert loads on caller routing (stack_fused_moe, as the reference's forward_cuda
calls it after select_experts, specmoe/layers/FusedMoE.py:174-196): every token on the same
two experts, one expert holding all tokens beside singletons, and a ragged token count, on the
weight-streaming kernels and on the MFMA-tiled kernels (many token ranges of one expert, the
last one ragged). Outputs against the oracle."""
import numpy as np
import pytest
import torch

from ae_amd import _lib
from ae_amd.layers import stack_fused_moe, tiled_min_tokens
from oracle import moe_ref as ref
from tests.helpers import TOL, f32_of, make_pool, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
H, I, E = 256, 128, 16


def _ids(kind, T, k):
    r = np.random.default_rng(T + k)
    if kind == "same_two":
        ids = np.tile(np.array([3, 11][:k] + list(range(k - 2)), dtype=np.int32), (T, 1))
    else:  # "hot": column 0 always expert 7, the others spread one token at a time
        ids = np.empty((T, k), dtype=np.int32)
        ids[:, 0] = 7
        for j in range(1, k):
            ids[:, j] = (np.arange(T) * 5 + j) % E
            ids[ids[:, j] == 7, j] = 8
    return ids, (r.random((T, k)) * 0.9 + 0.1).astype(np.float32)


@pytest.mark.parametrize("kind", ["same_two", "hot"])
@pytest.mark.parametrize("T,path", [(64, "streaming"), (1000, "streaming"), (1000, "tiled"),
                                    (4095, "tiled")])
def test_extreme_expert_loads(kind, T, path):
    k = 2
    ids, w = _ids(kind, T, k)
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    pool, slots = make_pool(E, H, I, BF, num_slots=E + 1, seed=T + 1)
    logits = torch.zeros((T, E), device=DEV, dtype=BF)
    with tiled_min_tokens(0 if path == "tiled" else 1 << 62):
        assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)["tiled"] == int(path == "tiled")
        y = stack_fused_moe(x.clone(), pool, slots, logits, torch.from_numpy(w).to(DEV),
                            torch.from_numpy(ids).to(DEV), False)
    torch.cuda.synchronize()
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(), w, ids, ref.BF16)
    parity(f32_of(y), y_ref, TOL[BF], case=f"{kind} T={T} {path}")
