"""CPU oracle for SpecMoE's verify-step MoE path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only to check results against (or as the timed CPU restatement in the baseline). The product path
(ae_amd) never imports it and has no CPU fallback.

A plain numpy restatement of the reference's arithmetic:

  routing   select_experts as called at specmoe/layers/FusedMoE.py:174-185 (sglang 0.4.5.post3
            -> sgl_kernel.topk_softmax, not vendored): fp32 softmax, top-k with ties to the
            lower expert index, optional w / sum(w). Grouped (use_grouped_topk): sglang's
            grouped_topk / biased_grouped_topk -- softmax or sigmoid + correction bias scores,
            only the topk_group best of num_expert_group groups selectable.
  align     moe_align_block_size, specmoe/layers/fused_moe_kernel.py:16-85 (sgl-kernel 0.1.2
            underneath, not vendored); pinned by the docstring example at :41-54.
  experts   stack_fused_moe, specmoe/layers/fused_moe_kernel.py:253-349: per routed
            assignment, C1 = round(x W13^T) (:332-335, rounded at :203), C2 =
            round(silu(C1_gate) * C1_up) (:337), C3 = round((C2 W2^T) * w) (:339-342, weight
            applied at :197-201), y = round(sum_j C3) (:344-347). round() is to the activation
            dtype; fp32 runs round nowhere by default. With fp16_outputs (fp32 only) the two
            GEMM outputs C1 and C3 are rounded to fp16 as the reference's Triton kernel
            stores them for fp32 inputs (compute_type fp16, :248; cast at :203), C2 stays fp32
            (silu_and_mul into the fp32 intermediate, :337) and so does the sum.
  page      FusedMoE.weight_loader, specmoe/layers/FusedMoE.py:485-505: one page per expert,
            [W1 (I x H) | W3 (I x H) | W2 (H x I)].
  norm      RMSNorm.forward_native, specmoe/layers/layernorm.py:36-52 (residual add in fp32,
            mean of squares, x * rsqrt(var + eps) * weight rounded once); router gate
            round(x W_g^T), specmoe/models/mixtral.py:84-91; called in order at :310-313.
  shared    no reference code (the reference serves only Mixtral). The MoE blocks of the
            public Qwen1.5-MoE / Qwen2-MoE and DeepSeek-V2 architectures, with the rounding
            points of their unfused layers: shared MLP d = round(round(silu(round(x W1s^T)) *
            round(x W3s^T)) W2s^T); Qwen gate s = round(sigmoid(gate logit)), shared term
            round(s * d); DeepSeek routed term round(y * routed_scaling_factor); block output
            round(routed term + shared term).

Routing arithmetic is restated operation for operation (same exp method, same summation
tree, correctly rounded fp32 divide), so GPU routing weights match this oracle bit for bit.
GEMM accumulation order is not restated; outputs agree to a stated tolerance.

Parity pinning (tests/test_oracle.py): the align docstring example; brute-force sorting;
top-k against np.argsort/lexsort selection and hand-built tie cases; the grouped top-k against
a Python sorted() re-derivation, the plain top-k where grouping removes nothing, hand-worked
cases (sigmoid_scores within 3 ulp of float64) and transformers' DeepSeek-V2 / V3 router
modules (the same picks and weights); exp_nonpos against float64
exp (<= 2 ulp); the expert math against a float64 textbook SwiGLU MoE built from separate
gate/up/down matrices through the page packing; the shared-expert block against a float64
textbook block and its reductions (zero shared page -> routed result, zero routed pages ->
dense MLP, saturated gate -> ungated / routed only). No reference test vectors exist beyond
the align docstring example (the reference ships no tests). Parity of the shared-expert block
with the reference is unpinned: the reference has no such block; it is pinned to the public
architectures, in fp32 against transformers' Qwen2MoeSparseMoeBlock and DeepseekV2Moe modules.
"""
from __future__ import annotations

import numpy as np

F32, F16, BF16 = "f32", "f16", "bf16"

_f32 = np.float32


def _c(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


# ---------------------------------------------------------------------------------------------
# dtype helpers: bf16/f16 values travel as float32 arrays holding representable values
# ---------------------------------------------------------------------------------------------
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (NaN stays a quiet NaN)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    r = np.where(nan, (u >> 16) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def round_to(a: np.ndarray, dtype: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dtype == BF16:
        return bf16_bits_to_f32(f32_to_bf16_bits(a))
    if dtype == F16:
        with np.errstate(over="ignore"):
            return a.astype(np.float16).astype(np.float32)
    if dtype == F32:
        return a
    raise ValueError(dtype)


def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    """Storage array (uint16 bits for bf16/f16, or float) -> float32 values."""
    a = np.asarray(a)
    if a.dtype == np.uint16:
        if dtype == BF16:
            return bf16_bits_to_f32(a)
        if dtype == F16:
            return a.view(np.float16).astype(np.float32)
        raise ValueError("uint16 storage needs dtype bf16 or f16")
    return a.astype(np.float32, copy=False)


# ---------------------------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------------------------
_LOG2E = _c(0x3FB8AA3B)
_C1 = _c(0x3F318000)  # 0.693359375, 9 significant bits
_C2 = _c(0xB95E8083)  # ln2 - C1
_P = [_c(0x39500D01), _c(0x3AB60B61), _c(0x3C088889), _c(0x3D2AAAAB), _c(0x3E2AAAAB),
      _f32(0.5), _f32(1.0), _f32(1.0)]  # 1/7! ... 1/2!, 1/1!, 1/0!


def exp_nonpos(d: np.ndarray) -> np.ndarray:
    """exp(d) for d <= 0 in float32: Cody-Waite reduction n = rint(d log2 e),
    r = (d - n C1) - n C2, degree-7 Taylor polynomial in Horner form, exact scale by 2^n;
    d < -80 gives 0, NaN gives NaN. Each operation is one IEEE fp32 multiply or add."""
    d = np.asarray(d, dtype=np.float32)
    out = np.zeros(d.shape, dtype=np.float32)
    ok = d >= _f32(-80.0)
    x = d[ok]
    n = np.rint(x * _LOG2E).astype(np.float32)
    r = (x - n * _C1) - n * _C2
    p = np.full_like(r, _P[0])
    for c in _P[1:]:
        p = p * r + c
    scale = ((n.astype(np.int32) + 127) << 23).astype(np.uint32).view(np.float32)
    out[ok] = p * scale
    nan = np.isnan(d)
    out[nan] = d[nan]
    return out


_LANES = 64
_PER_LANE = 4  # experts per lane (E <= 256)


def softmax_probs(logits: np.ndarray) -> np.ndarray:
    """fp32 softmax over the last axis with the kernel's summation order: expert e sits on
    lane e % 64 as its (e // 64)-th value; each lane sums its values in order, then lanes
    are combined pairwise by a butterfly with offsets 1, 2, 4, ..., 32 (lane l + lane l^1,
    then + lane l^2, ...). p = ex * (1 / sum)."""
    x = np.asarray(logits, dtype=np.float32)
    T, E = x.shape
    if E > _LANES * _PER_LANE:
        raise ValueError("E > 256")
    m = x.max(axis=1, keepdims=True)
    ex = exp_nonpos(x - m)
    pad = np.zeros((T, _LANES * _PER_LANE), dtype=np.float32)
    pad[:, :E] = ex
    lanes = pad.reshape(T, _PER_LANE, _LANES)
    s = lanes[:, 0, :].copy()
    for i in range(1, _PER_LANE):
        s = s + lanes[:, i, :]
    while s.shape[1] > 1:  # after each level the lanes of a pair hold equal values
        s = s[:, 0::2] + s[:, 1::2]
    inv = _f32(1.0) / s[:, 0]
    return ex * inv[:, None]


def topk_softmax(logits: np.ndarray, top_k: int, renormalize: bool):
    """-> (topk_weights float32 [T,k], topk_ids int32 [T,k]); ids in descending weight,
    ties to the lower expert index; renormalised by division by the in-order sum."""
    p = softmax_probs(logits)
    T, E = p.shape
    if not 1 <= top_k <= E:
        raise ValueError("top_k out of range")
    work = p.copy()
    rows = np.arange(T)
    w = np.empty((T, top_k), dtype=np.float32)
    ids = np.empty((T, top_k), dtype=np.int32)
    for j in range(top_k):
        idx = np.argmax(work, axis=1)  # first occurrence of the max = lowest index
        w[:, j] = work[rows, idx]
        ids[:, j] = idx
        work[rows, idx] = _f32(-1.0)
    if renormalize:
        s = w[:, 0].copy()
        for j in range(1, top_k):
            s = s + w[:, j]
        w = w / s[:, None]
    return w.astype(np.float32), ids


select_experts = topk_softmax


def sigmoid_scores(logits: np.ndarray) -> np.ndarray:
    """fp32 sigmoid with the routing exp: 1 / (1 + exp(-x)) for x >= 0, e / (1 + e) with
    e = exp(x) for x < 0 (exp_nonpos either way; each step one IEEE fp32 operation)."""
    x = np.asarray(logits, dtype=np.float32)
    pos = x >= _f32(0.0)
    e = exp_nonpos(np.where(pos, -x, x))
    one = _f32(1.0)
    out = np.empty_like(x)
    out[pos] = one / (one + e[pos])
    neg = ~pos
    out[neg] = e[neg] / (one + e[neg])
    return out


def grouped_topk(logits: np.ndarray, top_k: int, renormalize: bool, num_expert_group: int,
                 topk_group: int, correction_bias=None):
    """select_experts(use_grouped_topk=True) as called at specmoe/layers/FusedMoE.py:174-185:
    sglang 0.4.5.post3's grouped_topk (correction_bias None) and biased_grouped_topk (not
    vendored) -> (topk_weights float32 [T,k], topk_ids int32 [T,k]).

    Experts form num_expert_group groups of gs = E / num_expert_group consecutive experts.
    Scores s: softmax_probs (no bias) or sigmoid_scores (bias); choice c = s (+ bias). Group
    score: max of c over the group, or with a bias the sum of its two largest c. The
    topk_group best groups (descending score, ties to the lower group) stay selectable; the
    top_k best selectable experts by c (descending, ties to the lower expert) are the picks
    in that order, with weight s, renormalised by the in-order sum. NaN ranks as -inf.
    sglang's torch.topk(sorted=False) leaves the order of picks and of equal values open;
    this fixes both as the ungrouped top-k does."""
    x = np.asarray(logits, dtype=np.float32)
    T, E = x.shape
    ng, tg = int(num_expert_group), int(topk_group)
    if ng <= 0 or E % ng or not 1 <= tg <= ng:
        raise ValueError("bad expert groups")
    gs = E // ng
    if not 1 <= top_k <= tg * gs:
        raise ValueError("top_k out of range")
    if correction_bias is None:
        s = softmax_probs(x)
        c = s
    else:
        if gs < 2:
            raise ValueError("a biased group score needs two experts per group")
        s = sigmoid_scores(x)
        c = s + np.asarray(correction_bias, dtype=np.float32).reshape(1, E)
    c = np.where(np.isnan(c), _f32(-np.inf), c)
    cg = c.reshape(T, ng, gs)
    if correction_bias is None:
        gscore = cg.max(axis=2)
    else:
        top2 = np.sort(cg, axis=2)
        gscore = top2[:, :, -1] + top2[:, :, -2]
    gscore = np.where(np.isnan(gscore), _f32(-np.inf), gscore)
    rows = np.arange(T)[:, None]
    gorder = np.lexsort((np.broadcast_to(np.arange(ng), (T, ng)), -gscore), axis=-1)
    allowed = np.zeros((T, ng), dtype=bool)
    allowed[rows, gorder[:, :tg]] = True
    allowed = np.repeat(allowed, gs, axis=1)
    eorder = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -c, ~allowed), axis=-1)
    ids = eorder[:, :top_k].astype(np.int32)
    w = s[rows, ids].astype(np.float32)
    if renormalize:
        tot = w[:, 0].copy()
        for j in range(1, top_k):
            tot = tot + w[:, j]
        w = w / tot[:, None]
    return w.astype(np.float32), ids


# ---------------------------------------------------------------------------------------------
# alignment
# ---------------------------------------------------------------------------------------------
def expert_order(ids: np.ndarray, num_experts: int):
    """Stable expert sort of flat assignments: -> (counts [E], order [N']) where order lists
    the flat indices f of expert 0 (ascending), then expert 1, ...; ids outside [0,E) dropped."""
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    valid = (flat >= 0) & (flat < num_experts)
    counts = np.bincount(flat[valid], minlength=num_experts)
    keys = np.where(valid, flat, num_experts)
    order = np.argsort(keys, kind="stable")[: int(valid.sum())]
    return counts, order.astype(np.int32)


def moe_align_block_size(topk_ids: np.ndarray, block_size: int, num_experts: int):
    """Reference format: (sorted_ids [N + E*(BM-1)], expert_ids [cdiv(len, BM)], ntp [1]).
    Padding slots hold N; blocks past ntp/BM hold -1."""
    flat = np.asarray(topk_ids).reshape(-1)
    N = flat.size
    counts, order = expert_order(flat, num_experts)
    padded = (counts + block_size - 1) // block_size * block_size
    seg = np.concatenate([[0], np.cumsum(padded)]).astype(np.int64)
    length = N + num_experts * (block_size - 1)
    sorted_ids = np.full(length, N, dtype=np.int32)
    expert_ids = np.full((length + block_size - 1) // block_size, -1, dtype=np.int32)
    start = 0
    for e in range(num_experts):
        c = int(counts[e])
        sorted_ids[seg[e]:seg[e] + c] = order[start:start + c]
        expert_ids[seg[e] // block_size:seg[e + 1] // block_size] = e
        start += c
    return sorted_ids, expert_ids, np.array([seg[-1]], dtype=np.int32)


# ---------------------------------------------------------------------------------------------
# experts
# ---------------------------------------------------------------------------------------------
def pack_page(w1: np.ndarray, w3: np.ndarray, w2: np.ndarray) -> np.ndarray:
    """Page of one expert from HF-layout matrices: gate w1 [I,H], up w3 [I,H], down w2 [H,I]."""
    return np.concatenate([np.asarray(w1).reshape(-1), np.asarray(w3).reshape(-1),
                           np.asarray(w2).reshape(-1)])


def unpack_page(page: np.ndarray, H: int, dtype: str):
    """-> (W1 [I,H], W3 [I,H], W2 [H,I]) as float32."""
    page = np.asarray(page).reshape(-1)
    I = page.size // (3 * H)
    f = to_f32(page, dtype)
    return (f[: I * H].reshape(I, H), f[I * H: 2 * I * H].reshape(I, H),
            f[2 * I * H:].reshape(H, I))


def silu(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    return g / (_f32(1.0) + np.exp(-g))


def stack_fused_moe(x: np.ndarray, pool: np.ndarray, slots: np.ndarray, topk_weights: np.ndarray,
                    topk_ids: np.ndarray, dtype: str, num_experts: int | None = None,
                    fp16_outputs: bool = False) -> np.ndarray:
    """y [T,H] float32 (values representable in dtype). x and pool may be float arrays or
    uint16 bit arrays (bf16/f16). Assignments with an id outside [0,E) or a slot outside the
    pool contribute nothing. fp16_outputs (dtype f32 only): C1 and C3 rounded to fp16, as the
    reference stores fp32 runs' GEMM outputs (specmoe/layers/fused_moe_kernel.py:203,248)."""
    c_dt = F16 if (fp16_outputs and dtype == F32) else dtype
    xf = to_f32(x, dtype)
    T, H = xf.shape
    ids = np.asarray(topk_ids).reshape(T, -1)
    k = ids.shape[1]
    w = np.asarray(topk_weights, dtype=np.float32).reshape(T, k)
    slots = np.asarray(slots).reshape(-1)
    E = num_experts if num_experts is not None else slots.size
    P = pool.shape[0]
    c3 = np.zeros((T, k, H), dtype=np.float32)
    counts, order = expert_order(ids, E)
    start = 0
    for e in range(E):
        c = int(counts[e])
        f = order[start:start + c]
        start += c
        if c == 0:
            continue
        slot = int(slots[e])
        if not 0 <= slot < P:
            continue
        W1, W3, W2 = unpack_page(pool[slot], H, dtype)
        t, j = f // k, f % k
        xe = xf[t]
        g = round_to(xe @ W1.T, c_dt)
        u = round_to(xe @ W3.T, c_dt)
        a = round_to(silu(g) * u, dtype)
        d = (a @ W2.T) * w[t, j][:, None]
        c3[t, j] = round_to(d, c_dt)
    y = c3[:, 0, :].copy()
    for j in range(1, k):
        y = y + c3[:, j, :]
    return round_to(y, dtype)


def fused_moe_forward(x, router_logits, pool, slots, top_k: int, renormalize: bool, dtype: str,
                      fp16_outputs: bool = False):
    """FusedMoE.forward: routing then stack_fused_moe -> (y, topk_weights, topk_ids)."""
    logits = np.asarray(router_logits, dtype=np.float32)
    w, ids = topk_softmax(logits, top_k, renormalize)
    y = stack_fused_moe(x, pool, slots, w, ids, dtype, num_experts=logits.shape[1],
                        fp16_outputs=fp16_outputs)
    return y, w, ids


# ---------------------------------------------------------------------------------------------
# shared expert blocks (Qwen1.5-MoE / Qwen2-MoE, DeepSeek-V2); no reference counterpart
# ---------------------------------------------------------------------------------------------
def shared_expert_mlp(x: np.ndarray, page: np.ndarray, dtype: str) -> np.ndarray:
    """Dense SwiGLU MLP over every token with the weights of one page [W1s | W3s | W2s]:
    round(round(silu(round(x W1s^T)) * round(x W3s^T)) W2s^T) -> [T,H] float32."""
    xf = to_f32(x, dtype)
    W1, W3, W2 = unpack_page(page, xf.shape[1], dtype)
    g = round_to(xf @ W1.T, dtype)
    u = round_to(xf @ W3.T, dtype)
    a = round_to(silu(g) * u, dtype)
    return round_to(a @ W2.T, dtype)


def sigmoid(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, dtype=np.float32)
    with np.errstate(over="ignore"):  # exp(-z) = inf for z < -88.7: sigmoid = 0
        return _f32(1.0) / (_f32(1.0) + np.exp(-z))


def fused_moe_shared_forward(x, router_logits, pool, slots, top_k: int, renormalize: bool,
                             dtype: str, shared_page=None, shared_gate_logits=None,
                             routed_scaling_factor: float = 1.0):
    """The MoE block with a shared expert -> (y, topk_weights, topk_ids):
    y = round(round(routed * scale) + s * shared), s = round(sigmoid(gate logit)) or 1,
    the product s * shared rounded; routed = fused_moe_forward's result."""
    y, w, ids = fused_moe_forward(x, router_logits, pool, slots, top_k, renormalize, dtype)
    y = _block_terms(x, y, dtype, shared_page, shared_gate_logits, routed_scaling_factor)
    return y, w, ids


def stack_fused_moe_shared(x, pool, slots, topk_weights, topk_ids, dtype: str, shared_page=None,
                           shared_gate_logits=None, routed_scaling_factor: float = 1.0):
    """The same block on given routing (weights / ids as stack_fused_moe takes them)."""
    y = stack_fused_moe(x, pool, slots, topk_weights, topk_ids, dtype)
    return _block_terms(x, y, dtype, shared_page, shared_gate_logits, routed_scaling_factor)


def _block_terms(x, y, dtype: str, shared_page, shared_gate_logits, routed_scaling_factor: float):
    if routed_scaling_factor != 1.0:
        y = round_to(y * _f32(routed_scaling_factor), dtype)
    if shared_page is not None:
        d = shared_expert_mlp(x, shared_page, dtype)
        if shared_gate_logits is not None:
            sg = np.asarray(shared_gate_logits, dtype=np.float32).reshape(-1)
            s = round_to(sigmoid(sg), dtype)
            d = round_to(s[:, None] * d, dtype)
        y = round_to(y + d, dtype)
    return y


# ---------------------------------------------------------------------------------------------
# post-attention residual add + RMSNorm + router gate; the whole post-attention layer half
# ---------------------------------------------------------------------------------------------
def add_rmsnorm(x, residual, weight, eps: float, dtype: str):
    """RMSNorm.forward_native (specmoe/layers/layernorm.py:36-52) -> (normed, new_residual):
    s = fp32(x) [+ fp32(residual)], new_residual = round(s) (None without a residual),
    normed = round((s * (1 / sqrt(mean(s^2) + eps))) * weight). The mean of squares is taken
    exactly (float64) and rounded to fp32; the kernel's fp32 summation may differ from it in
    the last bits, so normed values agree to one rounding step."""
    s = to_f32(x, dtype)
    new_res = None
    if residual is not None:
        s = (s + to_f32(residual, dtype)).astype(np.float32)
        new_res = round_to(s, dtype)
    H = s.shape[-1]
    var = (np.square(s.astype(np.float64)).sum(axis=-1, keepdims=True) / H).astype(np.float32)
    rcp = (_f32(1.0) / np.sqrt(var + _f32(eps))).astype(np.float32)
    w = to_f32(weight, dtype).reshape(1, -1)
    return round_to((s * rcp) * w, dtype), new_res


def router_logits(xn, gate_weight, dtype: str):
    """The bias-free router gate (specmoe/models/mixtral.py:84-91): round(xn . W^T), fp32
    accumulation."""
    return round_to(to_f32(xn, dtype) @ to_f32(gate_weight, dtype).T, dtype)


def moe_layer_forward(x, residual, norm_weight, eps: float, gate_weight, pool, slots, top_k: int,
                      renormalize: bool, dtype: str, shared_page=None, shared_gate_weight=None,
                      routed_scaling_factor: float = 1.0, logits=None, shared_gate_logits=None):
    """Post-attention half of a MoE decoder layer (specmoe/models/mixtral.py:310-313) ->
    (y, new_residual, router_logits, topk_weights, topk_ids). `logits` / `shared_gate_logits`
    override the gate outputs (to route on given logit bits)."""
    xn, new_res = add_rmsnorm(x, residual, norm_weight, eps, dtype)
    lg = router_logits(xn, gate_weight, dtype) if logits is None else np.asarray(logits, np.float32)
    sgl = shared_gate_logits
    if sgl is None and shared_gate_weight is not None:
        sgl = router_logits(xn, np.asarray(shared_gate_weight).reshape(1, -1), dtype).reshape(-1)
    if shared_page is None and routed_scaling_factor == 1.0:
        y, w, ids = fused_moe_forward(xn, lg, pool, slots, top_k, renormalize, dtype)
    else:
        y, w, ids = fused_moe_shared_forward(xn, lg, pool, slots, top_k, renormalize, dtype,
                                             shared_page, sgl, routed_scaling_factor)
    return y, new_res, lg, w, ids
