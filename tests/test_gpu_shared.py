"""GPU parity of the MoE block with a shared expert (smx_fused_moe_shared_forward, and
smx_stack_fused_moe_shared on given routing) against the oracle, through the C ABI:
Qwen1.5-MoE-style gated shared expert, DeepSeek-V2-style ungated shared experts with a routed
scaling factor, the block modules, and DeepSeek-V2 / V3 grouped routing."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd import _lib
from ae_amd.layers import (DeepseekV2MoE, Qwen2MoeSparseMoeBlock, fused_moe_forward,
                           fused_moe_shared_forward, set_weight_attrs, stack_fused_moe_shared,
                           tiled_min_tokens)
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, parity, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, H, E, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(dtype)
    sgate = (torch.randn((T, 1), generator=g, device=DEV) * 2.0).to(dtype)
    return x, logits, sgate


def _shared_page(H, Is, dtype, seed, scale=0.02):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn((3 * Is * H,), generator=g, device=DEV) * scale).to(dtype)


def _oracle(x, logits, pool, slots, k, renorm, page, sgate, scale):
    dt = TORCH_TO_ORACLE[x.dtype]
    return ref.fused_moe_shared_forward(
        to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, renorm, dt,
        shared_page=None if page is None else to_oracle(page),
        shared_gate_logits=None if sgate is None else f32_of(sgate), routed_scaling_factor=scale)


def _check(x, logits, pool, slots, k, renorm, page, sgate, scale):
    y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, renorm, page, sgate,
                                         scale, inplace=False, return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle(x, logits, pool, slots, k, renorm, page, sgate, scale)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    T, H = x.shape
    parity(f32_of(y), y_ref, TOL[x.dtype],
           case=f"shared block T={T} H={H} I={pool.shape[1] // (3 * H)} E={logits.shape[1]} k={k} "
                f"Is={0 if page is None else page.numel() // (3 * H)} {x.dtype}")
    return y


CASES = [
    # T, H, I, E, k, Is
    (1, 128, 128, 4, 2, 256),
    (5, 256, 128, 8, 2, 384),
    (33, 256, 256, 16, 4, 128),
    (64, 128, 128, 8, 2, 512),
    (70, 256, 128, 8, 2, 256),     # two token ranges of the shared expert
    (130, 128, 256, 6, 3, 256),    # three token ranges
    (300, 256, 128, 8, 2, 256),    # five token ranges
]


# expert kernels: the weight-streaming ones or the tiled ones, forced either way
PATHS = {"streaming": 1 << 62, "tiled": 0}


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("T,H,I,E,k,Is", CASES)
def test_shared_block_matches_oracle(dtype, gated, T, H, I, E, k, Is, path):
    x, logits, sgate = _inputs(T, H, E, dtype, seed=T + Is)
    pool, slots = make_pool(E, H, I, dtype, num_slots=E + 2, seed=E + 1)
    page = _shared_page(H, Is, dtype, seed=Is)
    with tiled_min_tokens(PATHS[path]):
        _check(x, logits, pool, slots, k, gated, page, sgate if gated else None,
               1.0 if gated else 2.5)


def test_no_shared_expert_is_scaled_routed():
    T, H, I, E, k = 16, 256, 128, 8, 2
    x, logits, _ = _inputs(T, H, E, torch.bfloat16, seed=21)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=22)
    _check(x, logits, pool, slots, k, False, None, None, 16.0)
    y1 = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, None, None, 1.0,
                                  inplace=False)
    y2 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_qwen15_moe_shape():
    """Qwen1.5-MoE-A2.7B block: H 2048, 60 experts of I 1408, top-4 without renormalisation,
    gated shared expert of I 5632, 64 verify tokens; router logits 2*N(0,1)."""
    T, H, I, E, k, Is = 64, 2048, 1408, 60, 4, 5632
    x, logits, sgate = _inputs(T, H, E, torch.bfloat16, seed=31)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=32)
    page = _shared_page(H, Is, torch.bfloat16, seed=33)
    _check(x, logits, pool, slots, k, False, page, sgate, 1.0)


# The default plan's distinguishing features at each DeepSeek-V2-Lite verify size (so that
# every kernel form the stack runs is covered at its full shape).
DSV2_PLANS = {
    1: dict(fused_down=1, gateup_waves=4, gateup_ksplit=0),    # down + combine in one kernel
    2: dict(fused_down=1, gateup_waves=2, gateup_ksplit=0),    # 2-wave gate/up workgroups
    4: dict(fused_down=0, down_rows=1, gateup_ksplit=0),       # one W2 row tile per wave
    8: dict(fused_down=0, gateup_ksplit=1),                    # gate/up K split
    16: dict(fused_down=0, gateup_ksplit=1, down_rows=2),      # K split at full H = 2048
    32: dict(fused_down=0, gateup_ksplit=1, tok_tiles=2),
    64: dict(fused_down=0, gateup_ksplit=0, tok_tiles=4, down_rows=1),  # the row-tile rule
    128: dict(fused_down=0, tok_tiles=4, down_rows=1, shared_tok_groups=2),  # two token ranges
}


@pytest.mark.parametrize("T", sorted(DSV2_PLANS))
def test_deepseek_v2_lite_shape(T):
    """DeepSeek-V2-Lite block: H 2048, 64 experts of I 1408, top-6 without renormalisation,
    2 shared experts fused into one MLP of I 2816, routed scaling 1.0, on the default plan of
    each verify size (the plan's features asserted first)."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    plan = _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16, Is)
    assert plan["tiled"] == 0
    for key, want in DSV2_PLANS[T].items():
        assert plan[key] == want, (T, key, plan)
    x, logits, _ = _inputs(T, H, E, torch.bfloat16, seed=40 + T)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=41)
    page = _shared_page(H, Is, torch.bfloat16, seed=42)
    _check(x, logits, pool, slots, k, False, page, None, 1.0)


@pytest.mark.parametrize("T,L", [(1, 8), (4, 3)])
def test_deepseek_v2_lite_layer_chain_in_place(T, L):
    """L DeepSeek-V2-Lite blocks with distinct weights run in place one after another on one
    hidden-state buffer (each layer's output is the next one's input, as in the stack the
    benchmark times), against the oracle: every layer fed the GPU's input of that layer, and
    the whole chain fed its own outputs (L layers of 1e-2 each)."""
    H, I, E, k, Is = 2048, 1408, 64, 6, 2816
    x0, _, _ = _inputs(T, H, E, torch.bfloat16, seed=60 + T)
    layers = []
    for l in range(L):
        _, logits, _ = _inputs(T, H, E, torch.bfloat16, seed=70 + 10 * T + l)
        pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E, seed=80 + l)
        layers.append((logits, pool, slots, _shared_page(H, Is, torch.bfloat16, seed=90 + l)))
    buf = x0.clone()
    y_chain = to_oracle(x0)
    for l, (logits, pool, slots, page) in enumerate(layers):
        x_in = buf.clone()
        out = fused_moe_shared_forward(buf, logits, pool, slots, k, False, page, None, 1.0, inplace=True)
        torch.cuda.synchronize()
        assert out.data_ptr() == buf.data_ptr()
        y_ref, _, _ = _oracle(x_in, logits, pool, slots, k, False, page, None, 1.0)
        parity(f32_of(buf), y_ref, TOL[torch.bfloat16], case=f"dsv2lite chain T={T} layer {l}")
        y_chain, _, _ = ref.fused_moe_shared_forward(
            ref.f32_to_bf16_bits(y_chain) if y_chain.dtype != np.uint16 else y_chain,
            f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, False, "bf16",
            shared_page=to_oracle(page))
    parity(f32_of(buf), y_chain, L * TOL[torch.bfloat16], case=f"dsv2lite chain T={T} end to end",
           elementwise=False)


def test_shared_block_deterministic_bitwise():
    T, H, I, E, k, Is = 48, 256, 256, 8, 2, 512
    x, logits, sgate = _inputs(T, H, E, torch.bfloat16, seed=51)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=52)
    page = _shared_page(H, Is, torch.bfloat16, seed=53)
    outs = [fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, sgate,
                                     inplace=False) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def _load_block(block, E, H, I, Is, seed):
    g = torch.Generator().manual_seed(seed)
    dt = block.gate.weight.dtype
    with torch.no_grad():
        block.gate.weight.copy_(torch.randn(block.gate.weight.shape, generator=g) * 0.02)
        if block.shared_expert_gate is not None:
            block.shared_expert_gate.weight.copy_(torch.randn((1, H), generator=g) * 0.05)
    for e in range(E):
        for name, shape in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
            wt = (torch.randn(shape, generator=g) * 0.02).to(dt)
            block.experts.weight_loader(block.experts.ws, wt, f"experts.{e}.{name}.weight", name, e)
    gp, up = (torch.randn((Is, H), generator=g) * 0.02).to(dt), (torch.randn((Is, H), generator=g) * 0.02).to(dt)
    dp = (torch.randn((H, Is), generator=g) * 0.02).to(dt)
    block.load_shared_weights(gp, up, dp)
    block.to(DEV)
    pool = block.experts.ws.data.to(DEV)
    set_weight_attrs(block.experts.ws, {"gpu_cache": pool})
    return pool


@pytest.mark.parametrize("kind", ["qwen", "deepseek"])
def test_block_modules_end_to_end(kind):
    H, I, E, T = 256, 128, 8, 12
    if kind == "qwen":
        block = Qwen2MoeSparseMoeBlock(num_experts=E, top_k=4, hidden_size=H,
                                       moe_intermediate_size=I, shared_expert_intermediate_size=384,
                                       params_dtype=torch.bfloat16, tp_size=1)
        Is = 384
    else:
        block = DeepseekV2MoE(n_routed_experts=E, num_experts_per_tok=3, hidden_size=H,
                              moe_intermediate_size=I, n_shared_experts=2,
                              routed_scaling_factor=2.0, params_dtype=torch.bfloat16, tp_size=1)
        Is = 2 * I
    pool = _load_block(block, E, H, I, Is, seed=61)
    mapping = torch.arange(E, dtype=torch.int64, device=DEV)
    x = torch.randn((2, T // 2, H), generator=torch.Generator(device=DEV).manual_seed(62),
                    device=DEV).to(torch.bfloat16)
    x_in = x.clone()
    with torch.no_grad():
        logits = block.gate(x.view(-1, H))
        sg = block.shared_expert_gate(x.view(-1, H)) if kind == "qwen" else None
        y = block(x_in, mapping)
    torch.cuda.synchronize()
    assert y.shape == x.shape
    y_ref, _, _ = _oracle(x.view(-1, H), logits, pool, mapping, block.top_k, False,
                          block.shared_ws.data, sg, block.routed_scaling_factor)
    assert max_rel_err(f32_of(y.view(-1, H)), y_ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("shared", [False, True])
def test_hip_graph_replays_match_eager(shared):
    """The whole call captured in a HIP graph: every replay, with eager work and host
    synchronisations between replays, equals the eager result bit for bit."""
    T, H, I, E, k, Is = 20, 256, 128, 8, 2, 256
    x, logits, sgate = _inputs(T, H, E, torch.bfloat16, seed=71)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=72)
    page = _shared_page(H, Is, torch.bfloat16, seed=73) if shared else None
    out = torch.empty_like(x)

    def run():
        if shared:
            return fused_moe_shared_forward(x, logits, pool, slots, k, False, page, sgate,
                                            inplace=False)
        return fused_moe_forward(x, logits, pool, slots, k, True, inplace=False)

    eager = run()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.copy_(run())
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        run()  # eager work between replays
        torch.cuda.synchronize()


def test_shared_block_token_chunks():
    """DeepSeek-V2-style block (top-6, shared expert, routed scaling) with 3000 tokens = 18000
    assignments: two token chunks (2730 + 270) sharing one workspace."""
    T, H, I, E, k, Is = 3000, 128, 128, 16, 6, 256
    x, logits, _ = _inputs(T, H, E, torch.bfloat16, seed=94)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=95)
    page = _shared_page(H, Is, torch.bfloat16, seed=96)
    _check(x, logits, pool, slots, k, False, page, None, 2.5)


# ------------------------------------------------------- the block on the caller's routing
def _stack_shared(x, pool, slots, w, ids, page, sgate, scale):
    return stack_fused_moe_shared(x.clone(), pool, slots, w, ids, page, sgate, scale, inplace=False)


def _oracle_stack_shared(x, pool, slots, w, ids, page, sgate, scale):
    return ref.stack_fused_moe_shared(
        to_oracle(x), to_oracle(pool), slots.cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(),
        TORCH_TO_ORACLE[x.dtype], shared_page=None if page is None else to_oracle(page),
        shared_gate_logits=None if sgate is None else f32_of(sgate), routed_scaling_factor=scale)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,Is,gated", [(1, 128, 128, 8, 2, 256, True),
                                                (33, 256, 128, 16, 4, 384, False),
                                                (130, 128, 256, 6, 3, 256, True)])
def test_block_on_given_routing_equals_routed_block(dtype, T, H, I, E, k, Is, gated):
    """smx_stack_fused_moe_shared on the ids and weights smx_fused_moe_shared_forward chose gives
    that call's output bit for bit (same kernels), and matches the oracle's block."""
    x, logits, sgate = _inputs(T, H, E, dtype, seed=T + 3 * E)
    sgate = sgate if gated else None
    pool, slots = make_pool(E, H, I, dtype, num_slots=E + 2, seed=E + 1)
    page = _shared_page(H, Is, dtype, seed=Is)
    scale = 1.0 if gated else 2.5
    y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, True, page, sgate,
                                         scale, inplace=False, return_routing=True)
    y2 = _stack_shared(x, pool, slots, w, ids, page, sgate, scale)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    y_ref = _oracle_stack_shared(x, pool, slots, w, ids, page, sgate, scale)
    parity(f32_of(y2), y_ref, TOL[dtype], case=f"block on given routing T={T} E={E} k={k}")


def test_block_on_given_routing_token_chunks():
    """3000 tokens x top-6 = 18000 assignments: two token chunks, the shared gate logits of the
    second chunk offset with it."""
    T, H, I, E, k, Is = 3000, 128, 128, 16, 6, 256
    x, logits, sgate = _inputs(T, H, E, torch.bfloat16, seed=97)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=98)
    page = _shared_page(H, Is, torch.bfloat16, seed=99)
    w, ids = ref.grouped_topk(f32_of(logits), k, False, 4, 2)
    w_t, ids_t = torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    y = _stack_shared(x, pool, slots, w_t, ids_t, page, sgate, 1.0)
    torch.cuda.synchronize()
    y_ref = _oracle_stack_shared(x, pool, slots, w_t, ids_t, page, sgate, 1.0)
    parity(f32_of(y), y_ref, TOL[torch.bfloat16], case="block on given routing, token chunks")


@pytest.mark.parametrize("method,ng,tg,renorm,scale", [("group_limited_greedy", 8, 3, False, 16.0),
                                                       ("noaux_tc", 8, 4, True, 2.5),
                                                       ("noaux_tc", 1, 1, True, 1.0)])
@pytest.mark.parametrize("T", [1, 8, 64])
def test_deepseek_grouped_routing_blocks(method, ng, tg, renorm, scale, T):
    """DeepseekV2MoE with DeepSeek-V2's group-limited top-k and DeepSeek-V3's biased sigmoid
    top-k (reduced sizes: 64 routed experts of ffn 128, hidden 256, top-6 / top-8): the grouped
    top-k, then the block on that routing, against the oracle's grouped top-k and block."""
    H, I, E = 256, 128, 64
    k = 8 if method == "noaux_tc" else 6
    block = DeepseekV2MoE(n_routed_experts=E, num_experts_per_tok=k, hidden_size=H,
                          moe_intermediate_size=I, n_shared_experts=2, routed_scaling_factor=scale,
                          norm_topk_prob=renorm, params_dtype=torch.bfloat16, tp_size=1,
                          topk_method=method, n_group=ng, topk_group=tg)
    pool = _load_block(block, E, H, I, 2 * I, seed=71 + T)
    bias = getattr(block.gate, "e_score_correction_bias", None)
    if bias is not None:
        with torch.no_grad():
            bias.copy_(torch.randn(E, generator=torch.Generator().manual_seed(73)) * 0.05)
    mapping = torch.randperm(E, generator=torch.Generator().manual_seed(74)).to(DEV)
    x = torch.randn((T, H), generator=torch.Generator(device=DEV).manual_seed(75 + T),
                    device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        logits = block.gate(x)
        y = block(x.clone(), mapping)
    torch.cuda.synchronize()
    w_ref, ids_ref = ref.grouped_topk(f32_of(logits), k, renorm, ng, tg,
                                      None if bias is None else bias.detach().cpu().numpy())
    y_ref = ref.stack_fused_moe_shared(to_oracle(x), to_oracle(pool), mapping.cpu().numpy(), w_ref,
                                       ids_ref, ref.BF16, shared_page=to_oracle(block.shared_ws.data),
                                       routed_scaling_factor=scale)
    parity(f32_of(y), y_ref, TOL[torch.bfloat16], case=f"DeepseekV2MoE {method} T={T}")
    if method != "noaux_tc" or ng > 1:
        # the grouping (or the bias) is in effect: some token's picks differ from plain top-k
        assert T == 1 or (ids_ref != ref.topk_softmax(f32_of(logits), k, renorm)[1]).any()
