"""Host-side launch plans (smx_moe_plan_info, no GPU needed) of the down projection for the
measured shapes whose grid rules the kernels' timings were tuned on: the wave-target split,
the row-tile rule, and the wider grids for few assignments per expert on W2 rows that are not
a power-of-two number of bytes. A change to those rules shows here before it shows in a
benchmark."""
import pytest

from ae_amd import _lib

BF, F32 = _lib.SMX_BF16, _lib.SMX_F32

# (name, T, H, I, E, k, shared I, dtype) -> (K splits, W2 row tiles per wave)
CASES = [
    ("Mixtral-8x7B 1 token", 1, 4096, 14336, 8, 2, 0, BF, (8, 2)),
    ("Mixtral-8x7B 4 tokens: four residencies, 8 splits", 4, 4096, 14336, 8, 2, 0, BF, (8, 2)),
    ("Mixtral-8x7B 8 tokens", 8, 4096, 14336, 8, 2, 0, BF, (4, 2)),
    ("Mixtral-8x7B 32 tokens", 32, 4096, 14336, 8, 2, 0, BF, (2, 2)),
    ("Mixtral-8x22B 2 tokens: 32 KB rows keep two residencies", 2, 6144, 16384, 8, 2, 0, BF, (4, 2)),
    ("DBRX 1 token", 1, 6144, 10752, 16, 4, 0, BF, (4, 1)),
    ("fp32 layer of hidden 1024, 32 tokens", 32, 1024, 2816, 8, 2, 0, F32, (4, 1)),
    ("Qwen1.5-MoE 64 tokens", 64, 2048, 1408, 60, 4, 5632, BF, (1, 2)),
    ("DeepSeek-V2-Lite 32 tokens", 32, 2048, 1408, 64, 6, 2816, BF, (1, 2)),
    ("DeepSeek-V2-Lite 128 tokens", 128, 2048, 1408, 64, 6, 2816, BF, (1, 1)),
]


@pytest.mark.parametrize("name,T,H,I,E,k,Is,dt,want", CASES, ids=[c[0] for c in CASES])
def test_down_projection_plan(name, T, H, I, E, k, Is, dt, want):
    p = _lib.plan_info(T, H, I, E, k, dt, Is)
    assert p["tiled"] == 0, name
    assert (p["splits"], p["down_rows"]) == want, (name, p)
