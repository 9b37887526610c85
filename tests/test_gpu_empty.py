"""Empty batches (zero tokens) through every operator and module of the path: each returns
outputs of the right shapes, launches nothing that touches memory (the other buffers keep
their bits), and the next non-empty call on the same stream still matches the oracle. The
reference's operators take an empty batch the same way (torch ops over [0, H] tensors)."""
import numpy as np
import pytest
import torch

from ae_amd import _lib
from ae_amd.layers import (DeepseekV2MoE, MixtralMoE, PostAttentionMoE, Qwen2MoeSparseMoeBlock,
                           RMSNorm, add_rmsnorm_gate, fused_moe_forward, fused_moe_shared_forward,
                           grouped_topk, moe_align_block_size, moe_layer_forward, select_experts,
                           set_weight_attrs, stack_fused_moe, stack_fused_moe_shared)
from ae_amd.layers._torch import dtype_code, ptr, stream_of
from oracle import moe_ref as ref
from tests.helpers import TOL, f32_of, make_pool, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
H, I, E, K, IS = 256, 128, 16, 4, 256


def _empty(*shape, dtype=BF):
    return torch.empty(shape, device=DEV, dtype=dtype)


def _one_token_still_matches(pool, slots):
    """A one-token call after the empty ones: same stream, fresh routing, oracle parity."""
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn((1, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((1, E), generator=g, device=DEV) * 2.0).to(BF)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, K, True, inplace=False,
                                  return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(to_oracle(x), f32_of(logits), to_oracle(pool),
                                                  slots.cpu().numpy(), K, True, ref.BF16)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[BF]


def test_empty_batches_through_every_operator():
    pool, slots = make_pool(E, H, I, BF, num_slots=E + 2, seed=3)
    pool0 = pool.clone()
    page = (torch.randn((3 * IS * H,), device=DEV) * 0.02).to(BF)
    x, logits = _empty(0, H), _empty(0, E)

    w, ids = select_experts(x, logits, K, False, True)
    assert w.shape == (0, K) and ids.shape == (0, K)
    bias = torch.randn((E,), device=DEV)
    for b in (None, bias):
        w, ids = grouped_topk(logits, K, True, 4, 2, b)
        assert w.shape == (0, K) and ids.shape == (0, K)
    s, e, n = moe_align_block_size(_empty(0, K, dtype=torch.int32), 16, E)
    torch.cuda.synchronize()
    assert int(n.item()) == 0

    assert fused_moe_forward(x, logits, pool, slots, K, True).shape == (0, H)
    assert fused_moe_forward(x, logits, pool, slots, K, True, inplace=False).shape == (0, H)
    wt, it = _empty(0, K, dtype=torch.float32), _empty(0, K, dtype=torch.int32)
    assert stack_fused_moe(x, pool, slots, logits, wt, it, False).shape == (0, H)
    assert fused_moe_shared_forward(x, logits, pool, slots, K, False, page, _empty(0, 1), 1.0,
                                    inplace=False).shape == (0, H)
    assert stack_fused_moe_shared(x, pool, slots, wt, it, page, None, 2.5).shape == (0, H)

    # the allocation-free entry point, through the C ABI
    out = _empty(0, H)
    _lib.call("smx_fused_moe_forward_noalloc", ptr(x), ptr(out), dtype_code(BF), 0, H, ptr(logits),
              dtype_code(BF), E, K, 1, ptr(pool), pool.shape[0], pool.shape[1], ptr(slots), ptr(wt),
              ptr(it), stream_of(x))

    # residual add + RMSNorm (+ gate) and the whole post-attention layer call
    nw = torch.ones((H,), device=DEV, dtype=BF)
    gw = (torch.randn((E, H), device=DEV) * 0.05).to(BF)
    r = _empty(0, H)
    lg = add_rmsnorm_gate(x, r, nw, 1e-6, gw)
    assert lg.shape == (0, E)
    y, (lg, w, ids) = moe_layer_forward(x, r, nw, 1e-6, gw, pool, slots, K, True, shared_w=page,
                                        return_routing=True)
    assert y.shape == (0, H) and lg.shape == (0, E) and w.shape == (0, K) and ids.shape == (0, K)
    torch.cuda.synchronize()
    assert torch.equal(pool, pool0)
    _one_token_still_matches(pool, slots)


def _loaded(block, shared: bool):
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():
        block.gate.weight.copy_(torch.randn(block.gate.weight.shape, generator=g) * 0.05)
        block.experts.ws.copy_(torch.randn(block.experts.ws.shape, generator=g) * 0.02)
        if shared:
            block.shared_ws.copy_(torch.randn(block.shared_ws.shape, generator=g) * 0.02)
    block.to(DEV)
    set_weight_attrs(block.experts.ws, {"gpu_cache": block.experts.ws.data})
    return block


@pytest.mark.parametrize("kind", ["mixtral", "qwen", "deepseek_grouped"])
def test_empty_batches_through_the_modules(kind):
    """The block modules on [0, H] and [2, 0, H] inputs, alone and under PostAttentionMoE."""
    if kind == "mixtral":
        blk = _loaded(MixtralMoE(E, 2, H, I, params_dtype=BF, tp_size=1), False)
    elif kind == "qwen":
        blk = _loaded(Qwen2MoeSparseMoeBlock(num_experts=E, top_k=K, hidden_size=H,
                                             moe_intermediate_size=I, shared_expert_intermediate_size=IS,
                                             params_dtype=BF, tp_size=1), True)
    else:
        blk = _loaded(DeepseekV2MoE(n_routed_experts=E, num_experts_per_tok=K, hidden_size=H,
                                    moe_intermediate_size=I, n_shared_experts=2,
                                    routed_scaling_factor=2.0, topk_method="group_limited_greedy",
                                    n_group=4, topk_group=2, params_dtype=BF, tp_size=1), True)
    mapping = torch.arange(E, dtype=torch.int64, device=DEV)
    layer = PostAttentionMoE(RMSNorm(H).to(device=DEV, dtype=BF), blk)
    with torch.no_grad():
        for shape in ((0, H), (2, 0, H)):
            y = blk(_empty(*shape), mapping)
            assert y.shape == shape
            y, res = layer(_empty(*shape), _empty(*shape), mapping)
            assert y.shape == shape and res.shape == shape
        torch.cuda.synchronize()
        # a non-empty call afterwards: the residual of the norm run on its own, finite outputs
        # (the fused call's router logits come from its own gate kernel, so its routing is
        # compared with the oracle in the layer tests, not here); the grouped block's layer call
        # is the norm and then the block, bit for bit
        g = torch.Generator(device=DEV).manual_seed(12)
        x = torch.randn((3, H), generator=g, device=DEV).to(BF)
        r = torch.randn((3, H), generator=g, device=DEV).to(BF)
        y, res = layer(x.clone(), r.clone(), mapping)
        xs, rs = layer.post_attention_layernorm(x.clone(), r.clone())
        y2 = blk(xs, mapping)
    torch.cuda.synchronize()
    assert torch.equal(res, rs)
    assert bool(torch.isfinite(y).all()) and bool(torch.isfinite(y2).all())
    if kind == "deepseek_grouped":
        assert torch.equal(y, y2)
