"""GPU parity of the grouped top-k (smx_grouped_topk: sglang 0.4.5.post3's grouped_topk and
biased_grouped_topk, which select_experts runs for use_grouped_topk, reference call site
specmoe/layers/FusedMoE.py:174-185) against the oracle: bit-exact ids and weights; and
FusedMoE with grouped routing end to end (select_experts, then stack_fused_moe)."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import FusedMoE, select_experts, set_weight_attrs
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"

# E, groups, selected groups, k, biased
SHAPES = [
    (160, 8, 3, 6, False),   # DeepSeek-V2 (group-limited greedy)
    (256, 8, 4, 8, True),    # DeepSeek-V3 (sigmoid scores + correction bias)
    (64, 8, 2, 6, False), (64, 8, 2, 6, True),
    (8, 4, 2, 3, False), (8, 4, 2, 3, True),
    (60, 6, 1, 4, True), (96, 32, 5, 7, False), (128, 64, 16, 16, True),
    (200, 2, 1, 5, False), (256, 1, 1, 8, True), (12, 3, 3, 12, False),
]


def _route(logits, k, renorm, ng, tg, bias):
    w, ids = select_experts(torch.empty((logits.shape[0], 16), device=DEV), logits, k, True,
                            renorm, topk_group=tg, num_expert_group=ng, correction_bias=bias)
    torch.cuda.synchronize()
    return w.cpu().numpy(), ids.cpu().numpy()


def _oracle(logits, k, renorm, ng, tg, bias):
    b = None if bias is None else bias.float().cpu().numpy()
    return ref.grouped_topk(logits.float().cpu().numpy(), k, renorm, ng, tg, b)


def _check(logits, k, renorm, ng, tg, bias, case):
    w, ids = _route(logits, k, renorm, ng, tg, bias)
    w_ref, ids_ref = _oracle(logits, k, renorm, ng, tg, bias)
    np.testing.assert_array_equal(ids, ids_ref, err_msg=case)
    np.testing.assert_array_equal(w.view(np.uint32), w_ref.view(np.uint32), err_msg=case)
    return w, ids


@pytest.mark.parametrize("ldt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("E,ng,tg,k,biased", SHAPES)
@pytest.mark.parametrize("T", [1, 7, 130])
@pytest.mark.parametrize("renorm", [True, False])
def test_grouped_topk_bit_exact(ldt, E, ng, tg, k, biased, T, renorm):
    g = torch.Generator(device=DEV).manual_seed(T * 1000 + E * 10 + k + ng)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(ldt)
    bias = (torch.randn(E, generator=g, device=DEV) * 0.2) if biased else None
    _check(logits, k, renorm, ng, tg, bias, f"T={T} E={E} ng={ng} tg={tg} k={k} bias={biased}")


@pytest.mark.parametrize("biased", [False, True])
def test_grouped_topk_many_tokens(biased):
    """More tokens than the grid's waves (4096 workgroups of 4 waves): the waves walk the rest."""
    T, E, ng, tg, k = 20000, 160, 8, 3, 6
    g = torch.Generator(device=DEV).manual_seed(5 + int(biased))
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    bias = (torch.randn(E, generator=g, device=DEV) * 0.2) if biased else None
    _check(logits, k, True, ng, tg, bias, f"T={T} bias={biased}")


def test_grouped_topk_bf16_bias():
    """A bf16 correction bias (the model's parameter dtype) is read as its fp32 value."""
    T, E = 33, 256
    g = torch.Generator(device=DEV).manual_seed(9)
    logits = torch.randn((T, E), generator=g, device=DEV).to(torch.bfloat16)
    bias = (torch.randn(E, generator=g, device=DEV) * 0.2).to(torch.bfloat16)
    _check(logits, 8, True, 8, 4, bias, "bf16 bias")


def test_grouped_topk_known_answers():
    # softmax: group 3's best (1.45) loses to group 2's (1.5): expert 5 replaces expert 6
    x = torch.tensor([[0.0, 0.0, 2.0, -3.0, 1.5, 1.4, 1.45, 1.0]], device=DEV)
    _, ids = _check(x, 3, False, 4, 2, None, "softmax KAT")
    np.testing.assert_array_equal(ids[0], [2, 4, 5])
    # sigmoid + top-2 group sums: the group of the single best expert is not selected
    x = torch.tensor([[3.0, -5.0, 1.0, 1.0, 0.9, 0.9, -1.0, -1.0]], device=DEV)
    w, ids = _check(x, 2, True, 4, 2, torch.zeros(8, device=DEV), "sigmoid KAT")
    np.testing.assert_array_equal(ids[0], [2, 3])
    np.testing.assert_array_equal(w[0], [0.5, 0.5])
    # the bias steers the choice; the weight is the unbiased score
    x = torch.tensor([[2.0, 0.0, 1.0, 1.0]], device=DEV)
    bias = torch.tensor([0.0, 0.0, 0.5, 0.5], device=DEV)
    w, ids = _check(x, 1, False, 2, 1, bias, "bias KAT")
    assert ids[0, 0] == 2
    np.testing.assert_allclose(w[0, 0], 1.0 / (1.0 + np.exp(-1.0)), rtol=2e-7)


def test_grouped_topk_ties_and_extremes():
    x = torch.zeros((4, 16), device=DEV)
    x[1, [13, 2, 7]] = 1.0               # equal maxima in groups 0, 1, 3
    x[2] = -1e30                          # every exp but one underflows
    x[2, 9] = 0.0
    x[3] = torch.linspace(-200, 200, 16)  # sigmoid saturates at both ends
    for bias in (None, torch.zeros(16, device=DEV)):
        _, ids = _check(x, 3, False, 4, 2, bias, f"ties bias={bias is not None}")
        np.testing.assert_array_equal(ids[0], [0, 1, 2])
    _, ids = _check(x, 3, False, 4, 2, None, "ties")
    np.testing.assert_array_equal(ids[1], [2, 7, 0])


def test_fused_moe_grouped_routing_end_to_end():
    """FusedMoE(use_grouped_topk=True, ...) as the reference constructs it: the grouped top-k,
    then the experts on the pool, against the oracle's grouped top-k and expert math."""
    T, H, I, E, k, ng, tg = 24, 256, 256, 16, 4, 4, 2
    dtype = torch.bfloat16
    pool, slots = make_pool(E, H, I, dtype, num_slots=E + 3, seed=61)
    g = torch.Generator(device=DEV).manual_seed(62)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    for bias in (None, torch.randn(E, generator=g, device=DEV) * 0.3):
        moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I,
                       params_dtype=dtype, tp_size=1, use_grouped_topk=True, topk_group=tg,
                       num_expert_group=ng, correction_bias=bias)
        set_weight_attrs(moe.ws, {"gpu_cache": pool})
        out = moe(x.clone(), logits, slots)
        torch.cuda.synchronize()
        w_ref, ids_ref = _oracle(logits, k, True, ng, tg, bias)
        y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(), w_ref,
                                    ids_ref, TORCH_TO_ORACLE[dtype])
        parity(f32_of(out), y_ref, TOL[dtype], case=f"FusedMoE grouped bias={bias is not None}")
        # different picks from the ungrouped top-k on these inputs: the grouping is in effect
        assert (ids_ref != ref.topk_softmax(f32_of(logits), k, True)[1]).any()


def test_fused_moe_grouped_routing_tiled_sizes():
    """A prefill-sized batch (512 tokens, 16 experts, top-4: 128 expected tokens per expert, the
    MFMA-tiled expert kernels) through FusedMoE with the biased grouped top-k, against the
    oracle; the plan confirms the tiled kernels run."""
    from ae_amd import _lib
    T, H, I, E, k, ng, tg = 512, 256, 256, 16, 4, 4, 2
    dtype = torch.bfloat16
    assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)["tiled"] == 1
    pool, slots = make_pool(E, H, I, dtype, num_slots=E, seed=63)
    g = torch.Generator(device=DEV).manual_seed(64)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    bias = torch.randn(E, generator=g, device=DEV) * 0.3
    moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I, params_dtype=dtype,
                   tp_size=1, use_grouped_topk=True, topk_group=tg, num_expert_group=ng,
                   correction_bias=bias)
    set_weight_attrs(moe.ws, {"gpu_cache": pool})
    out = moe(x.clone(), logits, slots)
    torch.cuda.synchronize()
    w_ref, ids_ref = _oracle(logits, k, True, ng, tg, bias)
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(), w_ref, ids_ref,
                                TORCH_TO_ORACLE[dtype])
    parity(f32_of(out), y_ref, TOL[dtype], case="FusedMoE grouped, tiled sizes")


@pytest.mark.parametrize("T", [1, 8, 32])
def test_deepseek_v3_full_size_block(T):
    """The DeepSeek-V3 MoE block at full size: 256 routed experts (the library's maximum) of ffn
    2048, hidden 7168, the sigmoid top-8 with correction bias over 8 groups of which 4 stay
    selectable, renormalised, routed scaling 2.5, one shared expert of ffn 2048 -- the grouped
    top-k, then stack_fused_moe_shared on that routing. The 22.5 GB pool stays on the GPU; the
    oracle gets the picked experts' pages only (a compact pool and slot map)."""
    from ae_amd.layers import grouped_topk, stack_fused_moe_shared
    H, I, E, k, ng, tg, Is, scale = 7168, 2048, 256, 8, 8, 4, 2048, 2.5
    g = torch.Generator(device=DEV).manual_seed(500 + T)
    pool = torch.empty((E, 3 * I * H), dtype=torch.bfloat16, device=DEV)
    for e in range(E):
        pool[e].normal_(0.0, 0.02, generator=g)
    slots = torch.randperm(E, generator=torch.Generator().manual_seed(501)).to(DEV)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    bias = torch.randn((E,), generator=g, device=DEV) * 0.1
    w, ids = grouped_topk(logits, k, True, ng, tg, bias)
    y = stack_fused_moe_shared(x.clone(), pool, slots, w, ids, page, None, scale, inplace=False)
    torch.cuda.synchronize()
    w_ref, ids_ref = ref.grouped_topk(f32_of(logits), k, True, ng, tg, bias.cpu().numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    picked = np.unique(ids_ref)
    compact = to_oracle(pool[slots[torch.from_numpy(picked).to(DEV)]])
    cslots = np.full(E, -1, dtype=np.int64)
    cslots[picked] = np.arange(picked.size)
    del pool
    torch.cuda.empty_cache()
    y_ref = ref.stack_fused_moe_shared(to_oracle(x), compact, cslots, w_ref, ids_ref, ref.BF16,
                                       shared_page=to_oracle(page), routed_scaling_factor=scale)
    parity(f32_of(y), y_ref, TOL[torch.bfloat16], case=f"DeepSeek-V3 block T={T}")
