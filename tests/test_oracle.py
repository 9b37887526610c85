"""Pins the CPU oracle (oracle/moe_ref.py) with checks independent of its own formulas:
the reference's align docstring example, brute force, library selection routines, float64
exp/softmax, and a float64 textbook SwiGLU MoE built from separate gate/up/down matrices."""
import itertools
import json
import os

import numpy as np
import pytest

from oracle import moe_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# --------------------------------------------------------------------------------- dtype helpers
def test_bf16_rounding_known_values():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 2**-7, 1.0 + 3 * 2**-8, -2.5, 65504.0, 1e-40],
                    dtype=np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 is a tie -> even (1 + 2^-6)
    want = np.array([1.0, 1.0, 1.0 + 2**-7, 1.0 + 2**-6, -2.5, 65536.0, 0.0], dtype=np.float32)
    got = ref.round_to(vals, ref.BF16)
    np.testing.assert_array_equal(got[:6], want[:6])
    assert abs(got[6]) < 1e-39  # subnormal input rounds within the bf16 subnormal range


def test_bf16_round_matches_float64_nearest():
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(100000) * 10).astype(np.float32)
    got = ref.round_to(a, ref.BF16).astype(np.float64)
    # brute force: nearest of the two bf16 neighbours (truncate, truncate + 1 ulp)
    u = a.view(np.uint32)
    lo = (u & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((u & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    x = a.astype(np.float64)
    dlo, dhi = np.abs(x - lo), np.abs(hi - x)
    assert np.all(np.minimum(dlo, dhi) == np.abs(got - x))


def test_f16_round():
    a = np.array([1.0 + 2**-11, 1.0 + 3 * 2**-11, 70000.0], dtype=np.float32)
    np.testing.assert_array_equal(ref.round_to(a, ref.F16), [1.0, 1.0 + 2**-9, np.inf])


# ---------------------------------------------------------------------------------------- exp
def test_exp_nonpos_ulp_error():
    rng = np.random.default_rng(0)
    d = np.concatenate([
        -rng.random(2_000_000, dtype=np.float32) * np.float32(80.0),
        -rng.random(200_000, dtype=np.float32) * np.float32(1e-3),
        np.array([0.0, -0.0, -1e-30, -1e-7, -0.34657359, -0.34657360, -1.0, -79.999], np.float32),
    ]).astype(np.float32)
    got = ref.exp_nonpos(d)
    exact = np.exp(d.astype(np.float64))
    want = exact.astype(np.float32)
    ulp = np.spacing(want).astype(np.float64)
    err = np.abs(got.astype(np.float64) - exact) / ulp
    assert err.max() <= 2.0, err.max()
    assert ref.exp_nonpos(np.array([0.0], np.float32))[0] == 1.0


def test_exp_nonpos_edges():
    d = np.array([-80.0, -80.0001, -1000.0, -np.inf, np.nan], dtype=np.float32)
    out = ref.exp_nonpos(d)
    assert out[0] > 0 and np.isfinite(out[0])
    assert out[1] == 0 and out[2] == 0 and out[3] == 0
    assert np.isnan(out[4])
    # every nonzero result is a normal float
    assert out[0] >= np.finfo(np.float32).tiny


# ------------------------------------------------------------------------------------- softmax
def test_softmax_against_float64():
    rng = np.random.default_rng(2)
    for E in (1, 7, 8, 60, 64, 65, 128, 200, 256):
        x = (rng.standard_normal((33, E)) * 3).astype(np.float32)
        p = ref.softmax_probs(x)
        # the fp32 algorithm subtracts the row max in fp32; start float64 from those differences
        d32 = (x - x.max(1, keepdims=True)).astype(np.float32)
        e64 = np.exp(d32.astype(np.float64))
        p64 = e64 / e64.sum(1, keepdims=True)
        # exp (<= 2 ulp) + reciprocal + product + summation rounding: a few ulp
        np.testing.assert_allclose(p, p64, rtol=1e-6, atol=1e-30)
        np.testing.assert_allclose(p.sum(1), 1.0, rtol=2e-6)


def test_softmax_sum_order_is_the_lane_tree():
    # 70 experts: lanes 0..5 hold two values each. A sequential sum, a halving tree and the
    # lane butterfly differ for these magnitudes; the oracle must follow the butterfly (lane
    # sums, then lane l + lane l^1, then l^2, ... l^32).
    x = np.full((1, 70), -15.0, dtype=np.float32)
    x[0, 0] = 0.0
    x[0, 64] = -0.5
    ex = ref.exp_nonpos(x - x.max())
    pad = np.zeros(256, np.float32)
    pad[:70] = ex[0]
    lane = pad[:64].copy()
    for i in range(1, 4):
        lane = lane + pad[64 * i:64 * i + 64]
    tree = lane.copy()
    off = 1
    while off < 64:  # every lane of the butterfly, explicitly
        tree = tree + tree[np.arange(64) ^ off]
        off *= 2
    assert np.all(tree == tree[0])
    want = ex[0] * (np.float32(1.0) / tree[0])
    np.testing.assert_array_equal(ref.softmax_probs(x)[0], want)
    h, halving = 32, lane.copy()
    while h:
        halving = halving[:h] + halving[h:2 * h]
        h //= 2
    seq = np.float32(0)
    for v in ex[0]:
        seq = np.float32(seq + v)
    # the magnitudes make the three orders distinguishable
    assert len({float(tree[0]), float(halving[0]), float(seq)}) == 3


# --------------------------------------------------------------------------------------- top-k
def _select_by_lexsort(p, k):
    T, E = p.shape
    ids = np.empty((T, k), np.int32)
    for t in range(T):
        order = np.lexsort((np.arange(E), -p[t].astype(np.float64)))
        ids[t] = order[:k]
    return ids


@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (64, 6), (2, 2), (256, 8), (5, 1)])
def test_topk_matches_lexsort_selection(E, k):
    rng = np.random.default_rng(E * 10 + k)
    x = (rng.standard_normal((50, E)) * 2).astype(np.float32)
    p = ref.softmax_probs(x)
    w, ids = ref.topk_softmax(x, k, renormalize=False)
    np.testing.assert_array_equal(ids, _select_by_lexsort(p, k))
    np.testing.assert_array_equal(w, np.take_along_axis(p, ids.astype(np.int64), 1))
    assert np.all(np.diff(w, axis=1) <= 0)


def test_topk_ties_go_to_lower_index():
    x = np.zeros((3, 8), np.float32)
    x[1, [2, 5, 6]] = 1.0          # three-way tie at the top
    x[2] = [0, 3, 3, 1, 3, 0, 0, 1]
    w, ids = ref.topk_softmax(x, 3, renormalize=False)
    np.testing.assert_array_equal(ids[0], [0, 1, 2])
    np.testing.assert_array_equal(ids[1], [2, 5, 6])
    np.testing.assert_array_equal(ids[2], [1, 2, 4])
    assert w[0, 0] == w[0, 1] == w[0, 2] == np.float32(1.0) / np.float32(8.0)


def test_topk_renormalize_brute_force():
    # E=8, k=2: all 56 ordered pairs of distinct experts as the top two
    for a, b in itertools.permutations(range(8), 2):
        x = np.full((1, 8), -1.0, np.float32)
        x[0, a], x[0, b] = 2.0, 1.5
        w, ids = ref.topk_softmax(x, 2, renormalize=True)
        assert tuple(ids[0]) == (a, b)
        r = np.exp(0.5)
        np.testing.assert_allclose(w[0], [r / (1 + r), 1 / (1 + r)], rtol=2e-7)
        assert abs(float(w[0].sum(dtype=np.float64)) - 1.0) <= 2 * np.finfo(np.float32).eps


def test_topk_bf16_logits_select_like_logits():
    # bf16-representable logits that differ are never merged by the softmax: selecting on the
    # probabilities equals selecting on the logits (lexsort on logits, ties to lower index).
    rng = np.random.default_rng(7)
    x = ref.round_to((rng.standard_normal((400, 8)) * 1.3).astype(np.float32), ref.BF16)
    _, ids = ref.topk_softmax(x, 2, renormalize=True)
    np.testing.assert_array_equal(ids, _select_by_lexsort(x, 2))


# ------------------------------------------------------------------------------- grouped top-k
def test_sigmoid_scores_against_float64():
    rng = np.random.default_rng(11)
    x = np.concatenate([(rng.random(400_000, dtype=np.float32) - 0.5) * np.float32(160.0),
                        (rng.random(100_000, dtype=np.float32) - 0.5) * np.float32(1e-3),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 80.0, -80.0, 17.0, -17.0], np.float32)])
    got = ref.sigmoid_scores(x)
    exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - exact) / ulp
    assert err.max() <= 3.0, err.max()
    assert ref.sigmoid_scores(np.float32([0.0]))[0] == np.float32(0.5)
    edge = ref.sigmoid_scores(np.array([np.inf, -np.inf, -1000.0, 1000.0], np.float32))
    np.testing.assert_array_equal(edge, [1.0, 0.0, 0.0, 1.0])


def _grouped_by_python_sort(s, c, k, ng, tg, biased):
    """The grouped selection re-derived with Python's sorted() on tuple keys, token by token."""
    T, E = c.shape
    gs = E // ng
    ids = np.empty((T, k), np.int32)
    for t in range(T):
        row = [float(v) for v in c[t]]
        score = []
        for g in range(ng):
            members = row[g * gs:(g + 1) * gs]
            if biased:
                a, b = sorted(members)[-2:]
                score.append(float(np.float32(a) + np.float32(b)))
            else:
                score.append(max(members))
        groups = set(sorted(range(ng), key=lambda g: (-score[g], g))[:tg])
        cand = [e for e in range(E) if e // gs in groups]
        ids[t] = sorted(cand, key=lambda e: (-row[e], e))[:k]
    return ids


@pytest.mark.parametrize("E,ng,tg,k,biased", [(160, 8, 3, 6, False), (256, 8, 4, 8, True),
                                              (8, 4, 2, 3, False), (8, 4, 2, 3, True),
                                              (64, 8, 2, 6, False), (60, 6, 1, 4, True),
                                              (96, 32, 5, 7, False), (128, 64, 16, 16, True)])
def test_grouped_topk_against_python_sort(E, ng, tg, k, biased):
    rng = np.random.default_rng(E + 7 * ng + k + int(biased))
    x = (rng.standard_normal((40, E)) * 1.5).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32) if biased else None
    w, ids = ref.grouped_topk(x, k, False, ng, tg, bias)
    s = ref.sigmoid_scores(x) if biased else ref.softmax_probs(x)
    c = s + bias[None, :] if biased else s
    np.testing.assert_array_equal(ids, _grouped_by_python_sort(s, c, k, ng, tg, biased))
    np.testing.assert_array_equal(w, np.take_along_axis(s, ids.astype(np.int64), 1))
    # renormalised: the same picks, weights / their in-order sum
    wr, idr = ref.grouped_topk(x, k, True, ng, tg, bias)
    np.testing.assert_array_equal(idr, ids)
    np.testing.assert_allclose(wr.sum(axis=1, dtype=np.float64), 1.0, rtol=4e-7 * k)


@pytest.mark.parametrize("E,k", [(8, 2), (64, 6), (160, 6), (256, 8)])
def test_grouped_topk_reduces_to_plain_topk(E, k):
    # one group, or every group selectable: the plain top-k, bit for bit
    rng = np.random.default_rng(E + k)
    x = (rng.standard_normal((60, E)) * 2).astype(np.float32)
    for renorm in (False, True):
        w0, i0 = ref.topk_softmax(x, k, renorm)
        for ng, tg in ((1, 1), (8, 8), (4, 4)):
            if E % ng:
                continue
            w, ids = ref.grouped_topk(x, k, renorm, ng, tg)
            np.testing.assert_array_equal(ids, i0)
            np.testing.assert_array_equal(w.view(np.uint32), w0.view(np.uint32))


def test_grouped_topk_known_answers():
    # softmax, groups of 2: group 3's best (1.45) loses to group 2's (1.5), so expert 6 (the
    # plain top-3's third pick) is dropped for expert 5 of a selected group
    x = np.array([[0.0, 0.0, 2.0, -3.0, 1.5, 1.4, 1.45, 1.0]], np.float32)
    w, ids = ref.grouped_topk(x, 3, False, 4, 2)
    np.testing.assert_array_equal(ids[0], [2, 4, 5])
    np.testing.assert_array_equal(ref.topk_softmax(x, 3, False)[1][0], [2, 4, 6])
    p = np.exp(x[0].astype(np.float64))
    p /= p.sum()
    np.testing.assert_allclose(w[0], p[[2, 4, 5]], rtol=3e-7)
    # sigmoid + top-2 group sums: group 0 holds the single best expert (sigmoid(3)) but its
    # sum (0.9526 + 0.0067) loses to groups 1 (2 x 0.7311) and 2 (2 x 0.7109); equal picks
    # renormalise to exactly 1/2
    x = np.array([[3.0, -5.0, 1.0, 1.0, 0.9, 0.9, -1.0, -1.0]], np.float32)
    w, ids = ref.grouped_topk(x, 2, True, 4, 2, np.zeros(8, np.float32))
    np.testing.assert_array_equal(ids[0], [2, 3])
    np.testing.assert_array_equal(w[0], [0.5, 0.5])
    # the bias steers the choice, the weight stays the unbiased score
    x = np.array([[2.0, 0.0, 1.0, 1.0]], np.float32)
    bias = np.array([0.0, 0.0, 0.5, 0.5], np.float32)
    w, ids = ref.grouped_topk(x, 1, False, 2, 1, bias)
    assert ids[0, 0] == 2
    np.testing.assert_allclose(w[0, 0], 1.0 / (1.0 + np.exp(-1.0)), rtol=2e-7)
    w, ids = ref.grouped_topk(x, 1, True, 2, 1, bias)
    assert ids[0, 0] == 2 and w[0, 0] == np.float32(1.0)
    # equal logits: the lowest groups, then the lowest experts
    w, ids = ref.grouped_topk(np.zeros((1, 16), np.float32), 3, False, 4, 2)
    np.testing.assert_array_equal(ids[0], [0, 1, 2])


def test_grouped_topk_rejects_bad_groups():
    x = np.zeros((2, 12), np.float32)
    for ng, tg, k in ((5, 1, 1), (4, 5, 1), (4, 0, 1), (4, 1, 4), (12, 3, 1)):
        with pytest.raises(ValueError):
            ref.grouped_topk(x, k, False, ng, tg, np.zeros(12, np.float32) if ng == 12 else None)


# --------------------------------------------------------------------------------------- align
def test_align_docstring_example():
    """specmoe/layers/fused_moe_kernel.py:41-54 (read with expert 0 empty, E=5)."""
    with open(os.path.join(GOLDEN, "align_docstring_kat.json")) as f:
        kat = json.load(f)
    sorted_ids, expert_ids, ntp = ref.moe_align_block_size(
        np.array(kat["topk_ids"], np.int32), kat["block_size"], kat["num_experts"])
    np.testing.assert_array_equal(sorted_ids[:kat["num_tokens_post_pad"]], kat["sorted_token_ids"])
    assert int(ntp[0]) == kat["num_tokens_post_pad"]
    nb = kat["num_tokens_post_pad"] // kat["block_size"]
    np.testing.assert_array_equal(expert_ids[:nb], kat["expert_ids"])
    assert np.all(sorted_ids[kat["num_tokens_post_pad"]:] == len(sum(kat["topk_ids"], [])))


def _align_brute(flat, bm, E):
    out, eids = [], []
    for e in range(E):
        run = [f for f in range(len(flat)) if flat[f] == e]
        while len(run) % bm:
            run.append(len(flat))
        out += run
        eids += [e] * (len(run) // bm)
    return out, eids


@pytest.mark.parametrize("seed", range(12))
def test_align_brute_force(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 20))
    k = int(rng.integers(1, min(E, 6) + 1))
    T = int(rng.integers(0, 40))
    bm = int(rng.choice([1, 2, 4, 16, 64]))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if T else np.zeros((0, k), np.int32)
    flat = ids.reshape(-1).tolist()
    sorted_ids, expert_ids, ntp = ref.moe_align_block_size(ids, bm, E)
    want, weids = _align_brute(flat, bm, E)
    assert int(ntp[0]) == len(want)
    np.testing.assert_array_equal(sorted_ids[:len(want)], want)
    assert np.all(sorted_ids[len(want):] == len(flat))
    np.testing.assert_array_equal(expert_ids[:len(weids)], weids)
    assert np.all(expert_ids[len(weids):] == -1)
    # invariants: bijection onto [0, N) among non-sentinel entries
    real = sorted_ids[sorted_ids < len(flat)]
    np.testing.assert_array_equal(np.sort(real), np.arange(len(flat)))


# ---------------------------------------------------------------------------------- expert math
def _textbook(x, w1s, w3s, w2s, w, ids):
    """float64 Mixtral sparse MoE block: y = sum_j w_j * W2 (silu(W1 x) * (W3 x))."""
    x = x.astype(np.float64)
    y = np.zeros_like(x)
    for t in range(x.shape[0]):
        for j in range(ids.shape[1]):
            e = ids[t, j]
            g = w1s[e].astype(np.float64) @ x[t]
            u = w3s[e].astype(np.float64) @ x[t]
            a = g / (1 + np.exp(-g)) * u
            y[t] += w[t, j] * (w2s[e].astype(np.float64) @ a)
    return y


def _make_layer(rng, T, H, I, E, k, P, dtype):
    x = ref.round_to(rng.standard_normal((T, H)).astype(np.float32), dtype)
    w1s = [ref.round_to((rng.standard_normal((I, H)) * 0.05).astype(np.float32), dtype) for _ in range(E)]
    w3s = [ref.round_to((rng.standard_normal((I, H)) * 0.05).astype(np.float32), dtype) for _ in range(E)]
    w2s = [ref.round_to((rng.standard_normal((H, I)) * 0.05).astype(np.float32), dtype) for _ in range(E)]
    slots = rng.permutation(P)[:E]
    pool = np.zeros((P, 3 * I * H), np.float32)
    for e in range(E):
        pool[slots[e]] = ref.pack_page(w1s[e], w3s[e], w2s[e])
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    return x, w1s, w3s, w2s, slots, pool, logits


@pytest.mark.parametrize("dtype,rtol", [(ref.F32, 2e-5), (ref.BF16, 3e-2), (ref.F16, 4e-3)])
def test_expert_math_against_textbook(dtype, rtol):
    rng = np.random.default_rng(11)
    T, H, I, E, k = 9, 64, 96, 5, 2
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 8, dtype)
    y, w, ids = ref.fused_moe_forward(x, logits, pool, slots, k, True, dtype)
    want = _textbook(x, w1s, w3s, w2s, w, ids)
    err = np.abs(y - want).max() / np.abs(want).max()
    assert err < rtol, err


def _textbook_fp16_outputs(x, w1s, w3s, w2s, w, ids, round_act=False):
    """float64 block with the reference's fp32-input stores: gate/up outputs and the weighted
    down output cast to fp16 (np.float16, nearest even), activation and sum unrounded."""
    x = x.astype(np.float64)
    y = np.zeros_like(x)
    h16 = lambda v: v.astype(np.float16).astype(np.float64)
    for t in range(x.shape[0]):
        for j in range(ids.shape[1]):
            e = ids[t, j]
            g = h16(w1s[e].astype(np.float64) @ x[t])
            u = h16(w3s[e].astype(np.float64) @ x[t])
            a = g / (1 + np.exp(-g)) * u
            if round_act:
                a = h16(a)
            y[t] += h16(w[t, j] * (w2s[e].astype(np.float64) @ a))
    return y


def test_fp32_fp16_outputs_mode_against_textbook():
    """The opt-in fp16 stores of fp32 runs: close to the float64 block with fp16 casts at C1
    and C3 only, clearly farther from true fp32 and from a block that also rounds C2."""
    rng = np.random.default_rng(15)
    T, H, I, E, k = 8, 64, 96, 4, 2
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 6, ref.F32)
    y, w, ids = ref.fused_moe_forward(x, logits, pool, slots, k, True, ref.F32, fp16_outputs=True)
    y_plain, _, _ = ref.fused_moe_forward(x, logits, pool, slots, k, True, ref.F32)
    want = _textbook_fp16_outputs(x, w1s, w3s, w2s, w, ids)
    also_act = _textbook_fp16_outputs(x, w1s, w3s, w2s, w, ids, round_act=True)
    scale = np.abs(want).max()
    err = np.abs(y - want).max() / scale
    assert err < 2e-5, err
    assert np.abs(y_plain - want).max() / scale > 10 * err
    assert np.abs(y - also_act).max() / scale > 5 * err
    # a no-op for 16-bit activations
    xb = ref.round_to(x, ref.BF16)
    pb = ref.round_to(pool, ref.BF16)
    a1 = ref.stack_fused_moe(xb, pb, slots, w, ids, ref.BF16)
    a2 = ref.stack_fused_moe(xb, pb, slots, w, ids, ref.BF16, fp16_outputs=True)
    np.testing.assert_array_equal(a1, a2)


def test_expert_math_detects_swapped_gate_up():
    rng = np.random.default_rng(12)
    T, H, I, E, k = 6, 32, 64, 3, 2
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 3, ref.F32)
    y, w, ids = ref.fused_moe_forward(x, logits, pool, slots, k, True, ref.F32)
    swapped = _textbook(x, w3s, w1s, w2s, w, ids)
    assert np.abs(y - swapped).max() / np.abs(swapped).max() > 0.05


def test_single_expert_is_dense_swiglu():
    rng = np.random.default_rng(13)
    T, H, I = 4, 32, 64
    x, w1s, w3s, w2s, slots, pool, _ = _make_layer(rng, T, H, I, 1, 1, 1, ref.F32)
    y = ref.stack_fused_moe(x, pool, slots, np.ones((T, 1), np.float32),
                            np.zeros((T, 1), np.int32), ref.F32)
    g, u = x @ w1s[0].T, x @ w3s[0].T
    np.testing.assert_allclose(y, (g / (1 + np.exp(-g)) * u) @ w2s[0].T, rtol=1e-5, atol=1e-6)


def test_invalid_ids_and_slots_contribute_nothing():
    rng = np.random.default_rng(14)
    T, H, I, E, k = 4, 32, 64, 3, 2
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 4, ref.F32)
    w, ids = ref.topk_softmax(logits, k, True)
    base = ref.stack_fused_moe(x, pool, slots, w, ids, ref.F32)
    ids2 = ids.copy()
    ids2[:, 1] = 99
    y2 = ref.stack_fused_moe(x, pool, slots, w, ids2, ref.F32)
    w0 = w.copy()
    w0[:, 1] = 0
    y0 = ref.stack_fused_moe(x, pool, slots, w0, ids, ref.F32)
    assert np.abs(y2 - y0).max() <= 1e-5 * np.abs(y0).max()  # BLAS order differs with batch
    bad = slots.copy()
    bad[ids[0, 0]] = 1000
    y3 = ref.stack_fused_moe(x, pool, bad, w, ids, ref.F32)
    assert not np.allclose(y3, base)


# ------------------------------------------------------------------------ shared-expert blocks
def _textbook_block(x, w1s, w3s, w2s, w, ids, sg1, sg3, sg2, gate_w=None, scale=1.0):
    """float64 MoE block with a shared expert: scale * routed + s * W2s(silu(W1s x) * W3s x),
    s = sigmoid(gate_w . x) or 1."""
    y = _textbook(x, w1s, w3s, w2s, w, ids) * scale
    xd = x.astype(np.float64)
    g, u = xd @ sg1.T.astype(np.float64), xd @ sg3.T.astype(np.float64)
    d = (g / (1 + np.exp(-g)) * u) @ sg2.T.astype(np.float64)
    if gate_w is not None:
        d = d / (1 + np.exp(-(xd @ gate_w.astype(np.float64))))[:, None]
    return y + d


def _shared_mats(rng, H, Is, dtype):
    mk = lambda shape: ref.round_to((rng.standard_normal(shape) * 0.05).astype(np.float32), dtype)
    return mk((Is, H)), mk((Is, H)), mk((H, Is))


@pytest.mark.parametrize("dtype,rtol", [(ref.F32, 2e-5), (ref.BF16, 3e-2), (ref.F16, 4e-3)])
@pytest.mark.parametrize("gated", [True, False])
def test_shared_block_against_textbook(dtype, rtol, gated):
    rng = np.random.default_rng(21)
    T, H, I, E, k, Is = 7, 64, 32, 6, 3, 96
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 8, dtype)
    s1, s3, s2 = _shared_mats(rng, H, Is, dtype)
    gw = ref.round_to((rng.standard_normal(H) * 0.2).astype(np.float32), dtype) if gated else None
    sgl = ref.round_to(x @ gw, dtype) if gated else None
    scale = 1.0 if gated else 2.5
    y, w, ids = ref.fused_moe_shared_forward(x, logits, pool, slots, k, False, dtype,
                                             ref.pack_page(s1, s3, s2), sgl, scale)
    want = _textbook_block(x, w1s, w3s, w2s, w, ids, s1, s3, s2, gw, scale)
    err = np.abs(y - want).max() / np.abs(want).max()
    assert err < rtol, err
    # a swapped shared gate/up or a dropped gate is far outside the tolerance
    bad = _textbook_block(x, w1s, w3s, w2s, w, ids, s3, s1, s2, gw, scale)
    assert np.abs(y - bad).max() / np.abs(bad).max() > 0.05
    if gated:
        ungated = _textbook_block(x, w1s, w3s, w2s, w, ids, s1, s3, s2, None, scale)
        assert np.abs(y - ungated).max() / np.abs(ungated).max() > 0.05


def test_shared_block_reductions():
    """Zero shared page -> the routed result; zero routed pages -> the dense shared MLP;
    a saturated gate logit -> gate 1 (ungated) or 0 (routed only)."""
    rng = np.random.default_rng(22)
    T, H, I, E, k, Is = 6, 64, 32, 4, 2, 64
    dt = ref.BF16
    x, w1s, w3s, w2s, slots, pool, logits = _make_layer(rng, T, H, I, E, k, 4, dt)
    s1, s3, s2 = _shared_mats(rng, H, Is, dt)
    page = ref.pack_page(s1, s3, s2)
    routed, _, _ = ref.fused_moe_forward(x, logits, pool, slots, k, False, dt)
    y0, _, _ = ref.fused_moe_shared_forward(x, logits, pool, slots, k, False, dt,
                                            np.zeros_like(page), None, 1.0)
    np.testing.assert_array_equal(y0, routed)
    dense = ref.shared_expert_mlp(x, page, dt)
    y1, _, _ = ref.fused_moe_shared_forward(x, logits, np.zeros_like(pool), slots, k, False, dt,
                                            page, None, 1.0)
    np.testing.assert_array_equal(y1, dense)
    g, u = x @ s1.T, x @ s3.T
    np.testing.assert_allclose(dense, (g / (1 + np.exp(-g)) * u) @ s2.T, rtol=3e-2,
                               atol=3e-2 * np.abs(dense).max())
    ungated, _, _ = ref.fused_moe_shared_forward(x, logits, pool, slots, k, False, dt, page, None)
    hi, _, _ = ref.fused_moe_shared_forward(x, logits, pool, slots, k, False, dt, page,
                                            np.full(T, 100.0, np.float32))
    np.testing.assert_array_equal(hi, ungated)
    lo, _, _ = ref.fused_moe_shared_forward(x, logits, pool, slots, k, False, dt, page,
                                            np.full(T, -100.0, np.float32))
    np.testing.assert_array_equal(lo, routed)


# ----------------------------------------------------------------- residual add + RMSNorm + gate
def _bf16(a):
    return ref.f32_to_bf16_bits(np.asarray(a, np.float32))


def test_add_rmsnorm_against_torch_native_formula():
    """The reference's forward_native (layernorm.py:36-52) is torch arithmetic; evaluate it with
    torch on the CPU (its own reduction order and rsqrt) and compare: the residual is exact,
    the normalized values agree to one bf16 rounding step."""
    import torch
    rng = np.random.default_rng(31)
    T, H, eps = 7, 512, 1e-6
    x, r = _bf16(rng.standard_normal((T, H)) * 3), _bf16(rng.standard_normal((T, H)))
    w = _bf16(1 + 0.1 * rng.standard_normal(H))
    xn, res = ref.add_rmsnorm(x, r, w, eps, ref.BF16)
    tx = torch.from_numpy(ref.to_f32(x, ref.BF16)).to(torch.bfloat16)
    tr = torch.from_numpy(ref.to_f32(r, ref.BF16)).to(torch.bfloat16)
    tw = torch.from_numpy(ref.to_f32(w, ref.BF16)).to(torch.bfloat16)
    s = tx.to(torch.float32) + tr.to(torch.float32)
    t_res = s.to(torch.bfloat16)
    var = s.pow(2).mean(dim=-1, keepdim=True)
    t_xn = ((s * torch.rsqrt(var + eps)) * tw).to(torch.bfloat16)
    np.testing.assert_array_equal(res, t_res.float().numpy())
    ulp = np.abs(ref.f32_to_bf16_bits(xn).astype(np.int64) -
                 t_xn.view(torch.int16).numpy().astype(np.uint16).astype(np.int64))
    assert ulp.max() <= 1 and (ulp > 0).mean() < 0.01


def test_rmsnorm_unit_rms_and_float64():
    rng = np.random.default_rng(32)
    T, H, eps = 5, 1024, 1e-5
    x = (rng.standard_normal((T, H)) * 7).astype(np.float32)
    xn, res = ref.add_rmsnorm(x, None, np.ones(H, np.float32), eps, ref.F32)
    assert res is None
    rms = np.sqrt(np.mean(xn.astype(np.float64) ** 2, axis=-1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-5)
    w = rng.standard_normal(H).astype(np.float32)
    xn2, _ = ref.add_rmsnorm(x, None, w, eps, ref.F32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps) * w
    np.testing.assert_allclose(xn2, want, rtol=2e-6, atol=2e-6 * np.abs(want).max())


def test_router_logits_and_layer_composition():
    """The layer restatement is norm -> gate -> MoE: with the logits given it equals the MoE
    oracle applied to the normalized states; the gate matches a float64 product."""
    rng = np.random.default_rng(33)
    T, H, I, E, k = 6, 64, 32, 4, 2
    dt = ref.BF16
    x, r = _bf16(rng.standard_normal((T, H))), _bf16(rng.standard_normal((T, H)))
    nw = _bf16(np.ones(H))
    gw = _bf16(rng.standard_normal((E, H)) * 0.2)
    pool = _bf16(rng.standard_normal((E, 3 * I * H)) * 0.05)
    slots = np.arange(E)
    y, res, lg, w, ids = ref.moe_layer_forward(x, r, nw, 1e-6, gw, pool, slots, k, True, dt)
    xn, res2 = ref.add_rmsnorm(x, r, nw, 1e-6, dt)
    np.testing.assert_array_equal(res, res2)
    want = xn.astype(np.float64) @ ref.to_f32(gw, dt).T.astype(np.float64)
    assert np.abs(lg - want).max() <= 8e-3 * np.abs(want).max()
    y2, w2, ids2 = ref.fused_moe_forward(ref.f32_to_bf16_bits(xn), lg, pool, slots, k, True, dt)
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(ids, ids2)


def _hf_deepseek_router(version, E, k, ng, tg, renorm, bias):
    """transformers' DeepSeek-V2 / V3 router modules (an independent implementation of the same
    routing) with an identity gate, so that their logits are the given ones exactly."""
    pytest.importorskip("transformers")
    import torch
    from types import SimpleNamespace
    if version == 2:
        from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2TopkRouter
        cfg = SimpleNamespace(num_experts_per_tok=k, num_experts=E, hidden_size=E,
                              routed_scaling_factor=1.0, topk_method="group_limited_greedy",
                              n_group=ng, topk_group=tg)
        r = DeepseekV2TopkRouter(cfg)
    else:
        from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter
        cfg = SimpleNamespace(num_experts_per_tok=k, num_local_experts=E, hidden_size=E,
                              routed_scaling_factor=1.0, n_group=ng, topk_group=tg,
                              norm_topk_prob=renorm)
        r = DeepseekV3TopkRouter(cfg)
        r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    with torch.no_grad():
        r.weight.copy_(torch.eye(E))
    return r


@pytest.mark.parametrize("version,E,ng,tg,k,renorm", [(2, 160, 8, 3, 6, False), (2, 64, 8, 2, 6, False),
                                                      (2, 16, 4, 2, 3, False), (3, 256, 8, 4, 8, True),
                                                      (3, 64, 8, 2, 6, True), (3, 32, 4, 1, 4, False)])
def test_grouped_topk_against_transformers_deepseek_routers(version, E, ng, tg, k, renorm):
    """The grouped top-k against transformers' DeepseekV2TopkRouter (group-limited greedy:
    softmax, group max) and DeepseekV3TopkRouter (sigmoid + correction bias, top-2 group sums):
    the same experts for every token (their torch.topk(sorted=False) leaves the order open, so
    picks are compared as sets) and the same weight per expert, to fp32 rounding (torch's exp
    and, for V3, its +1e-20 in the renormalising sum)."""
    import torch
    rng = np.random.default_rng(E + 10 * version + k)
    T = 64
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if version == 3 else None
    router = _hf_deepseek_router(version, E, k, ng, tg, renorm, bias)
    with torch.no_grad():
        hf_logits, w_hf, ids_hf = router(torch.from_numpy(logits))
    np.testing.assert_array_equal(hf_logits.numpy(), logits)  # the identity gate is exact
    w, ids = ref.grouped_topk(logits, k, renorm, ng, tg, bias)
    ids_hf = ids_hf.numpy()
    w_hf = w_hf.numpy()
    for t in range(T):
        assert sorted(ids[t].tolist()) == sorted(ids_hf[t].tolist()), t
        by_id = dict(zip(ids_hf[t].tolist(), w_hf[t].tolist()))
        np.testing.assert_allclose(w[t], [by_id[e] for e in ids[t].tolist()], rtol=3e-6, atol=0)


@pytest.mark.parametrize("kind", ["qwen2_moe", "deepseek_v2_greedy", "deepseek_v2_grouped"])
def test_shared_block_against_transformers_modules(kind):
    """The shared-expert block (and, for DeepSeek-V2, its group-limited routing) against
    transformers' Qwen2MoeSparseMoeBlock and DeepseekV2Moe in fp32, an independent
    implementation of the public architectures: the oracle in fp32 (no rounding points) on the
    same weights, packed into pool pages and a shared page, agrees to fp32 summation order."""
    pytest.importorskip("transformers")
    import torch
    from transformers import DeepseekV2Config, Qwen2MoeConfig
    torch.manual_seed(3)
    T, H, I, E, k = 12, 128, 64, 16, 4
    if kind == "qwen2_moe":
        from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeSparseMoeBlock
        cfg = Qwen2MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                             moe_intermediate_size=I, shared_expert_intermediate_size=192,
                             norm_topk_prob=False)
        blk = Qwen2MoeSparseMoeBlock(cfg).float()
        router_w, shared, scale, ng, tg = blk.gate.weight, blk.shared_expert, 1.0, 1, 1
    else:
        from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2Moe
        grouped = kind.endswith("grouped")
        cfg = DeepseekV2Config(hidden_size=H, n_routed_experts=E, num_experts_per_tok=k,
                               moe_intermediate_size=I, n_shared_experts=2,
                               n_group=4 if grouped else 1, topk_group=2 if grouped else 1,
                               topk_method="group_limited_greedy" if grouped else "greedy",
                               routed_scaling_factor=2.0, hidden_act="silu")
        blk = DeepseekV2Moe(cfg).float()
        router_w, shared, scale = blk.gate.weight, blk.shared_experts, 2.0
        ng, tg = (4, 2) if grouped else (1, 1)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape) * 0.05)
        x = torch.randn((1, T, H))
        y_hf = blk(x).reshape(T, H).numpy()
    xs = x.reshape(T, H).numpy()
    logits = (xs.astype(np.float64) @ router_w.detach().numpy().T.astype(np.float64)).astype(np.float32)
    gu = blk.experts.gate_up_proj.detach().numpy()   # [E, 2I, H]: gate rows, then up rows
    dn = blk.experts.down_proj.detach().numpy()      # [E, H, I]
    pool = np.concatenate([gu.reshape(E, -1), dn.reshape(E, -1)], axis=1)  # [W1 | W3 | W2]
    page_s = np.concatenate([shared.gate_proj.weight.detach().numpy().reshape(-1),
                             shared.up_proj.weight.detach().numpy().reshape(-1),
                             shared.down_proj.weight.detach().numpy().reshape(-1)])
    sgl = None
    if kind == "qwen2_moe":
        sgl = (xs.astype(np.float64) @ blk.shared_expert_gate.weight.detach().numpy().T).astype(np.float32)
    w, ids = ref.grouped_topk(logits, k, False, ng, tg)
    y = ref.stack_fused_moe_shared(xs, pool, np.arange(E), w, ids, ref.F32, shared_page=page_s,
                                   shared_gate_logits=sgl, routed_scaling_factor=scale)
    err = np.abs(y - y_hf).max() / np.abs(y_hf).max()
    assert err < 2e-5, err


def test_routed_layer_against_transformers_mixtral_block():
    """The routed layer (FusedMoE's math: softmax top-2, renormalised, SwiGLU experts over pool
    pages) against transformers' MixtralSparseMoeBlock in fp32 -- the public implementation of
    the reference's model (specmoe/models/mixtral.py:59-115) -- on the same weights."""
    pytest.importorskip("transformers")
    import torch
    from transformers import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
    torch.manual_seed(4)
    T, H, I, E, k = 20, 128, 96 * 2, 8, 2
    cfg = MixtralConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k)
    blk = MixtralSparseMoeBlock(cfg).float().eval()
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape) * 0.05)
        x = torch.randn((1, T, H))
        y_hf = blk(x).reshape(T, H).numpy()
    xs = x.reshape(T, H).numpy()
    logits = (xs.astype(np.float64) @ blk.gate.weight.detach().numpy().T.astype(np.float64)).astype(np.float32)
    gu = blk.experts.gate_up_proj.detach().numpy()
    dn = blk.experts.down_proj.detach().numpy()
    pool = np.concatenate([gu.reshape(E, -1), dn.reshape(E, -1)], axis=1)
    slots = np.array([3, 0, 7, 1, 6, 2, 5, 4])  # through a permuted slot map
    y, _, _ = ref.fused_moe_forward(xs, logits, pool[np.argsort(slots)], slots, k, True, ref.F32)
    err = np.abs(y - y_hf).max() / np.abs(y_hf).max()
    assert err < 2e-5, err
