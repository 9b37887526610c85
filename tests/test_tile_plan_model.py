"""CPU check of the tiled expert path's work decomposition: for many routings -- the Mixtral
layer at 256 and 1024 tokens under Zipf-skewed gates, routings that pile every token onto two
experts, range counts at and just past a multiple of 128, dropped assignments, shared experts
over several token ranges, and the small shapes the GPU tests force onto the tiled path --
every act row and every partial that a kernel reads was written exactly once by an earlier
kernel of the call (tests/tile_plan_model.py restates the device-side decomposition; grids,
splits and spans come from the library's own host plan)."""
import contextlib

import numpy as np
import pytest

from ae_amd import _lib
from tests.tile_plan_model import check_tiled_coverage, range_group

EB = {_lib.SMX_BF16: 2, _lib.SMX_F16: 2, _lib.SMX_F32: 4}


@contextlib.contextmanager
def tiled_threshold(tokens):
    lib = _lib.lib()
    prev = int(lib.smx_tiled_min_tokens())
    lib.smx_set_tiled_min_tokens(-1 if tokens is None else tokens)
    try:
        yield
    finally:
        lib.smx_set_tiled_min_tokens(prev)


def _topk(logits: np.ndarray, k: int) -> np.ndarray:
    return np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int64)


def _zipf_logits(T, H, E, seed, s=1.2):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H), dtype=np.float32)
    wg = rng.standard_normal((E, H), dtype=np.float32) * 0.02
    p = np.arange(1, E + 1, dtype=np.float64) ** (-s)
    return x @ wg.T + np.log(p / p.sum()).astype(np.float32)


def _check(T, H, I, E, k, dtype, ids, routable=None, Is=0):
    plan = _lib.plan_info(T, H, I, E, k, dtype, Is)
    if routable is None:
        routable = np.ones_like(ids, dtype=bool)
    return check_tiled_coverage(T, H, I, k, EB[dtype], ids, routable, E, plan, Is=Is)


def test_range_group_is_a_bijection():
    for per_item in (1, 3, 8, 12, 16, 112, 113):
        for nr in (1, 2, 3, 5):
            seen = {range_group(local, per_item, nr) for local in range(per_item * nr)}
            assert seen == {(r, g) for r in range(nr) for g in range(per_item)}


@pytest.mark.parametrize("T", [256, 1024])
def test_mixtral_zipf_default_threshold(T):
    H, I, E, k = 4096, 14336, 8, 2
    with tiled_threshold(None):
        assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)["tiled"] == 1
        for seed in range(6 if T == 256 else 2):
            ids = _topk(_zipf_logits(T, H, E, seed=T + seed), k)
            stats = _check(T, H, I, E, k, _lib.SMX_BF16, ids)
            assert stats["ranges"] >= 8


def test_mixtral_every_token_on_two_experts():
    """The densest routing: experts 0 and 1 take all 256 tokens (two full ranges each)."""
    H, I, E, k, T = 4096, 14336, 8, 2, 256
    ids = np.tile(np.array([[0, 1]]), (T, 1))
    with tiled_threshold(None):
        assert _check(T, H, I, E, k, _lib.SMX_BF16, ids)["ranges"] == 4


@pytest.mark.parametrize("per_expert", [127, 128, 129, 255, 256, 257])
def test_range_counts_at_multiples_of_128(per_expert):
    """Every expert holds exactly per_expert assignments (k = 1 routing over 4 experts)."""
    H, I, E, k = 256, 256, 4, 1
    T = 4 * per_expert
    ids = np.repeat(np.arange(E), per_expert)[:, None]
    with tiled_threshold(0):
        _check(T, H, I, E, k, _lib.SMX_BF16, ids)


CASES = [
    # T, H, I, E, k  (the shapes the GPU tests force onto the tiled path)
    (1, 128, 128, 4, 2), (16, 128, 128, 4, 2), (33, 384, 256, 8, 2), (130, 256, 128, 3, 3),
    (300, 128, 256, 4, 2), (520, 256, 128, 16, 4), (64, 256, 384, 64, 6), (384, 256, 256, 8, 2),
]


@pytest.mark.parametrize("dtype", [_lib.SMX_BF16, _lib.SMX_F32])
@pytest.mark.parametrize("T,H,I,E,k", CASES)
def test_forced_tiled_shapes(dtype, T, H, I, E, k):
    rng = np.random.default_rng(T * 7 + E)
    with tiled_threshold(0):
        for _ in range(3):
            ids = _topk(rng.standard_normal((T, E)) * 2.0, k)
            _check(T, H, I, E, k, dtype, ids)


@pytest.mark.parametrize("I", [64, 192])
def test_fp32_partial_column_groups(I):
    rng = np.random.default_rng(I)
    with tiled_threshold(0):
        _check(200, 128, I, 4, 2, _lib.SMX_F32, _topk(rng.standard_normal((200, 4)), 2))


def test_dropped_assignments():
    """Assignments to unmapped experts are left out of the records; their partials are never
    computed and the combine does not read them."""
    T, H, I, E, k = 300, 256, 128, 8, 2
    rng = np.random.default_rng(3)
    ids = _topk(rng.standard_normal((T, E)), k)
    routable = ~np.isin(ids, [2, 5])
    with tiled_threshold(0):
        _check(T, H, I, E, k, _lib.SMX_BF16, ids, routable)


@pytest.mark.parametrize("T,H,I,E,k,Is", [(5, 256, 128, 8, 2, 384), (130, 128, 256, 6, 3, 256),
                                          (300, 256, 128, 8, 2, 640), (200, 256, 256, 8, 2, 512)])
@pytest.mark.parametrize("dtype", [_lib.SMX_BF16, _lib.SMX_F32])
def test_shared_expert_ranges(T, H, I, E, k, Is, dtype):
    rng = np.random.default_rng(T + Is)
    with tiled_threshold(0):
        _check(T, H, I, E, k, dtype, _topk(rng.standard_normal((T, E)), k), Is=Is)


def test_model_catches_a_missing_range():
    """The check fails when the grid is one range short (a planted plan error)."""
    T, H, I, E, k = 300, 128, 256, 4, 2
    ids = np.repeat(np.arange(E), T * k // E).reshape(T, k)
    with tiled_threshold(0):
        plan = _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)
    short = dict(plan)
    short["max_ranges"] = 4  # the routing needs 8 (150 assignments per expert: 2 ranges each)
    short["tile_gateup_grid"] = plan["tile_gateup_grid"] - (plan["max_ranges"] - 4) * (I // 128)
    short["tile_down_grid"] = plan["tile_down_grid"] - (plan["max_ranges"] - 4) * (H // 256) * plan["splits"]
    with pytest.raises(AssertionError):
        check_tiled_coverage(T, H, I, k, 2, ids, np.ones_like(ids, dtype=bool), E, short)
