"""GPU parity of the MoE layer entry points (stack_fused_moe, FusedMoE.forward / the fused
routing+experts call, MixtralMoE) against the oracle, through the C ABI."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import (FusedMoE, MixtralMoE, fused_moe_forward, select_experts,
                           set_weight_attrs, stack_fused_moe, tiled_min_tokens)
from tests.helpers import (TOL, TORCH_TO_ORACLE, f32_of, make_pool, max_rel_err, parity, to_oracle,
                           zipf_gate_logits)

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


CASES = [
    # T, H, I, E, k, slots
    (1, 128, 128, 4, 2, 4),
    (5, 256, 384, 8, 2, 16),
    (33, 256, 128, 8, 2, 8),
    (64, 128, 256, 16, 4, 20),
    (70, 128, 128, 8, 2, 8),      # > 64 tokens on one expert: several token groups
    (130, 256, 128, 3, 3, 3),     # every expert sees every token
    # up to 64 assignments over up to 64 experts in up to 4 top-k passes: routed by one wave
    (1, 256, 128, 64, 6, 64),
    (4, 256, 128, 64, 6, 70),
    (8, 128, 128, 32, 8, 32),     # exactly 64 assignments
    (3, 128, 128, 60, 16, 60),
    (8, 256, 128, 64, 6, 70),     # 8 passes: the multi-wave kernel
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,P", CASES)
def test_fused_forward_matches_oracle(dtype, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T + H + I)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                  return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    err = max_rel_err(f32_of(y), y_ref)
    assert err <= TOL[dtype], err


# Large batches on the streaming kernels (forced: several of these reach the tiled kernels'
# threshold): experts with several 64-token ranges (run side by side on one XCD).
LARGE_CASES = [
    # T, H, I, E, k, slots
    (256, 256, 128, 8, 2, 8),
    (300, 128, 256, 4, 2, 6),      # ragged last range of every expert
    (520, 256, 128, 16, 4, 20),
    (257, 128, 128, 3, 3, 3),      # every expert sees every token: 3 ranges each
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H,I,E,k,P", LARGE_CASES)
def test_large_batch_matches_oracle(dtype, T, H, I, E, k, P):
    x, logits = _inputs(T, H, E, dtype, seed=T + H + I)
    pool, slots = make_pool(E, H, I, dtype, num_slots=P, seed=E)
    with tiled_min_tokens(1 << 62):
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                      return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    err = max_rel_err(f32_of(y), y_ref)
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_stack_fused_moe_inplace_matches_oracle(dtype):
    T, H, I, E, k = 24, 256, 256, 8, 2
    x, logits = _inputs(T, H, E, dtype, seed=3)
    pool, slots = make_pool(E, H, I, dtype, num_slots=2 * E, seed=4)
    w, ids = select_experts(x, logits, k, False, True)
    x_in = x.clone()
    out = stack_fused_moe(x_in, pool, slots, logits, w, ids, True, inplace=True)
    torch.cuda.synchronize()
    assert out.data_ptr() == x_in.data_ptr()
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), TORCH_TO_ORACLE[dtype])
    assert max_rel_err(f32_of(out), y_ref) <= TOL[dtype]


def test_reference_operator_index_map():
    """The reference's own operator harness maps 8 experts onto a 16-slot pool through
    [0,2,3,6,8,10,12,14] (specmoe/optimizer/performance_simulator/operators/gpu_fused_moe.py:26-27)."""
    T, H, I, E, k = 16, 256, 256, 8, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=9)
    pool, _ = make_pool(E, H, I, torch.bfloat16, num_slots=16, seed=10)
    slots = torch.tensor([0, 2, 3, 6, 8, 10, 12, 14], dtype=torch.int64, device=DEV)
    y = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    y_ref, _, _ = _oracle_forward(x, logits, pool, slots, k, True)
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.bfloat16]


def test_only_mapped_pages_are_read():
    """Pages outside the map may hold anything (the H2D engine writes them concurrently)."""
    T, H, I, E, k = 16, 128, 128, 4, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=11)
    pool, _ = make_pool(E, H, I, torch.bfloat16, num_slots=8, seed=12)
    slots = torch.tensor([1, 3, 5, 7], dtype=torch.int64, device=DEV)
    y1 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    pool[[0, 2, 4, 6]] = float("nan")
    y2 = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_invalid_slot_contributes_nothing():
    T, H, I, E, k = 16, 128, 128, 4, 2
    x, logits = _inputs(T, H, E, torch.float32, seed=13)
    pool, slots = make_pool(E, H, I, torch.float32, seed=14)
    slots[1] = 99  # outside the pool
    y = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
    y_ref, _, _ = _oracle_forward(x, logits, pool, slots, k, True)
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.float32]


def test_deterministic_bitwise():
    T, H, I, E, k = 48, 256, 256, 8, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=15)
    pool, slots = make_pool(E, H, I, torch.bfloat16, seed=16)
    outs = [fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
            for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def test_zero_tokens():
    x = torch.empty((0, 128), device=DEV, dtype=torch.bfloat16)
    logits = torch.empty((0, 4), device=DEV, dtype=torch.bfloat16)
    pool, slots = make_pool(4, 128, 128, torch.bfloat16)
    y = fused_moe_forward(x, logits, pool, slots, 2, True)
    assert y.shape == (0, 128)


def test_fused_moe_module_end_to_end():
    """FusedMoE built and loaded like the reference (weight_loader from HF-layout matrices,
    pool attached as ws.gpu_cache), forward in place."""
    T, H, I, E, k = 12, 256, 256, 8, 2
    dtype = torch.bfloat16
    moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I,
                   params_dtype=dtype, tp_size=1)
    g = torch.Generator().manual_seed(21)
    for e in range(E):
        for name, shape in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
            wt = (torch.randn(shape, generator=g) * 0.05).to(dtype)
            moe.weight_loader(moe.ws, wt, f"experts.{e}.{name}.weight", name, e)
    pool = torch.zeros((2 * E, 3 * I * H), dtype=dtype, device=DEV)
    mapping = torch.arange(E, 2 * E, dtype=torch.int64, device=DEV).flip(0)
    pool[mapping.cpu()] = moe.ws.data.to(DEV)
    set_weight_attrs(moe.ws, {"gpu_cache": pool})
    x, logits = _inputs(T, H, E, dtype, seed=22)
    x_in = x.clone()
    out = moe(x_in, logits, mapping)
    torch.cuda.synchronize()
    assert out.data_ptr() == x_in.data_ptr()
    y_ref, _, _ = _oracle_forward(x, logits, pool, mapping, k, True)
    assert max_rel_err(f32_of(out), y_ref) <= TOL[dtype]


def test_fused_moe_routed_scaling_factor_accepted():
    """FusedMoE(routed_scaling_factor=2.5), as the reference's constructor allows, runs. The
    factor reaches select_experts only (reference FusedMoE.py:184), whose ungrouped top-k
    (sglang 0.4.5.post3 fused_topk) does not use it: the output equals the layer without it and
    the oracle's routed MoE with unscaled weights."""
    T, H, I, E, k = 20, 256, 256, 8, 2
    dtype = torch.bfloat16
    pool, slots = make_pool(E, H, I, dtype, num_slots=E, seed=23)
    x, logits = _inputs(T, H, E, dtype, seed=24)
    outs = []
    for factor in (None, 2.5):
        moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I,
                       params_dtype=dtype, tp_size=1, routed_scaling_factor=factor)
        set_weight_attrs(moe.ws, {"gpu_cache": pool})
        outs.append(moe(x.clone(), logits, slots))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    y_ref, _, _ = _oracle_forward(x, logits, pool, slots, k, True)
    parity(f32_of(outs[1]), y_ref, TOL[dtype], case="FusedMoE routed_scaling_factor=2.5")


def test_fused_moe_ignored_options_give_the_default_output():
    """FusedMoE built with the options the reference's forward_cuda ignores
    (activation="gelu", apply_router_weight_on_input=True, inplace=False, no_combine=True)
    computes what the reference computes for them: the default SiLU, combined, in-place
    output."""
    import warnings
    T, H, I, E, k = 9, 256, 256, 8, 2
    dtype = torch.bfloat16
    pool, slots = make_pool(E, H, I, dtype, num_slots=E, seed=25)
    x, logits = _inputs(T, H, E, dtype, seed=26)
    outs = []
    for opts in ({}, dict(activation="gelu", apply_router_weight_on_input=True, inplace=False,
                          no_combine=True)):
        moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I,
                       params_dtype=dtype, tp_size=1, **opts)
        set_weight_attrs(moe.ws, {"gpu_cache": pool})
        x_in = x.clone()
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", RuntimeWarning)
            out = moe(x_in, logits, slots)
        assert out.data_ptr() == x_in.data_ptr()
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_mixtral_moe_block():
    T, H, I, E, k = 10, 256, 128, 8, 2
    dtype = torch.bfloat16
    blk = MixtralMoE(E, k, H, I, params_dtype=dtype, tp_size=1).to(DEV)
    torch.nn.init.normal_(blk.gate.weight, std=0.05)
    pool, slots = make_pool(E, H, I, dtype, seed=31)
    set_weight_attrs(blk.experts.ws, {"gpu_cache": pool})
    x = torch.randn((2, T // 2, H), device=DEV).to(dtype)
    logits = torch.nn.functional.linear(x.view(-1, H), blk.gate.weight)
    y_ref, _, _ = _oracle_forward(x.view(-1, H), logits, pool, slots, k, True)
    out = blk(x.clone(), slots)
    torch.cuda.synchronize()
    assert out.shape == x.shape
    assert max_rel_err(f32_of(out.view(-1, H)), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("T,H,I,E,k,renorm", [
    (64, 2048, 1408, 60, 4, False),    # Qwen1.5-MoE-A2.7B routed experts
    (16, 2048, 1408, 64, 6, False),    # DeepSeek-V2-Lite routed experts
    (128, 2048, 1408, 64, 6, False),
])
def test_other_model_shapes(T, H, I, E, k, renorm):
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=T + E)
    pool, slots = make_pool(E, H, I, dtype, seed=41)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, renorm, inplace=False,
                                  return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[dtype]


@pytest.mark.parametrize("path", ["default", "tiled"])
def test_cpu_reference_config(path):
    """The reference's CPU-runnable configuration: hidden 1024, ffn 2816, 8 experts, top-2, fp32,
    32 tokens (4 sequences x 8 draft tokens) of N(0,1) hidden states, gate and expert weights
    N(0, 0.02), seed 0; the router logits are x Wg^T. On the default plan (weight-streaming
    kernels at 8 tokens per expert) and with the tiled kernels forced."""
    T, H, I, E, k = 32, 1024, 2816, 8, 2
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn((T, H), generator=g, device=DEV)
    wg = torch.randn((E, H), generator=g, device=DEV) * 0.02
    logits = x @ wg.T
    pool, slots = make_pool(E, H, I, torch.float32, seed=0)
    with tiled_min_tokens(0 if path == "tiled" else None):
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                      return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.float32]


@pytest.mark.parametrize("T", [1, 4, 8, 32, 64])
def test_mixtral_full_size(T):
    """Mixtral-8x7B MoE layer (H=4096, I=14336, E=8, top-2, bf16) with the Zipf-skewed gate, on
    the default plan of each batch size (T=1: fused down + combine; T=4: split down kernel with
    one W2 row tile per wave; T=32 and 64: routing inside the gate/up launch)."""
    H, I, E, k = 4096, 14336, 8, 2
    dtype = torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(100 + T)
    x = torch.randn((T, H), generator=g, device=DEV).to(dtype)
    logits = zipf_gate_logits(x, E, seed=T)
    pool, slots = make_pool(E, H, I, dtype, seed=7)
    y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                  return_routing=True)
    torch.cuda.synchronize()
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
    del pool
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    parity(f32_of(y), y_ref, TOL[dtype], case=f"mixtral full size T={T}")


@pytest.mark.parametrize("inplace", [False, True])
def test_more_than_16384_assignments_run_in_token_chunks(inplace):
    """T*top_k above the expert sort's 16384: the call runs as consecutive token chunks (8192
    tokens at top-2) sharing one workspace; routing and outputs match the oracle on every token."""
    T, H, I, E, k = 9000, 128, 128, 8, 2
    x, logits = _inputs(T, H, E, torch.bfloat16, seed=90)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=10, seed=91)
    x_in = x.clone()
    y, w, ids = fused_moe_forward(x_in, logits, pool, slots, k, True, inplace=inplace,
                                  return_routing=True)
    torch.cuda.synchronize()
    assert (y.data_ptr() == x_in.data_ptr()) == inplace
    y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.bfloat16]


def test_stack_fused_moe_token_chunks():
    T, H, I, E, k = 9000, 128, 256, 8, 2
    x, logits = _inputs(T, H, E, torch.float16, seed=92)
    pool, slots = make_pool(E, H, I, torch.float16, seed=93)
    w, ids = select_experts(x, logits, k, False, True)
    out = stack_fused_moe(x.clone(), pool, slots, logits, w, ids, True, inplace=False)
    torch.cuda.synchronize()
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.cpu().numpy(), ids.cpu().numpy(), TORCH_TO_ORACLE[torch.float16])
    assert max_rel_err(f32_of(out), y_ref) <= TOL[torch.float16]


def test_fused_moe_custom_routing_function():
    """FusedMoE with a caller-supplied routing function: its weights and ids drive the experts
    (reference FusedMoE.py:174-196), checked against the oracle's expert math on them."""
    T, H, I, E, k = 40, 256, 256, 8, 2
    dtype = torch.bfloat16

    def route(hidden_states, gating_output, topk, renormalize):
        # the k lowest-logit experts, weights 1/k (any rule the caller likes)
        ids = torch.argsort(gating_output.float(), dim=-1)[:, :topk]
        return torch.full(ids.shape, 1.0 / topk, device=ids.device), ids

    moe = FusedMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I,
                   params_dtype=dtype, tp_size=1, custom_routing_function=route)
    pool, slots = make_pool(E, H, I, dtype, num_slots=2 * E, seed=51)
    set_weight_attrs(moe.ws, {"gpu_cache": pool})
    x, logits = _inputs(T, H, E, dtype, seed=52)
    out = moe(x.clone(), logits, slots)
    torch.cuda.synchronize()
    w, ids = route(x, logits, k, True)
    y_ref = ref.stack_fused_moe(to_oracle(x), to_oracle(pool), slots.cpu().numpy(),
                                w.float().cpu().numpy(), ids.int().cpu().numpy(), TORCH_TO_ORACLE[dtype])
    assert max_rel_err(f32_of(out), y_ref) <= TOL[dtype]


# Work items in XCD order (every active expert one range, >= 32 ranges, >= 8 items per range):
# shapes where the order applies, with and without a shared expert (whose leading workgroups
# shift the routed ones off a multiple of 8), and one where the grid has no spare range (top-1,
# 40 tokens over 64 experts) so the launch keeps the plain order.
@pytest.mark.parametrize("T,E,k,Is", [(64, 64, 6, 0), (128, 64, 6, 0), (128, 60, 4, 1536),
                                      (40, 64, 1, 0), (96, 48, 3, 512)])
def test_many_single_range_experts(T, E, k, Is):
    from ae_amd.layers import fused_moe_shared_forward
    H, I = 512, 512
    dtype = torch.bfloat16
    x, logits = _inputs(T, H, E, dtype, seed=T * 3 + E + k)
    pool, slots = make_pool(E, H, I, dtype, seed=E + Is)
    if Is:
        g = torch.Generator(device=DEV).manual_seed(T + Is)
        page = (torch.randn(3 * Is * H, generator=g, device=DEV) * 0.02).to(dtype)
        y, _, _ = fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.0,
                                           inplace=False, return_routing=True)
        torch.cuda.synchronize()
        y_ref, _, _ = ref.fused_moe_shared_forward(
            to_oracle(x), f32_of(logits), to_oracle(pool), slots.cpu().numpy(), k, False, "bf16",
            shared_page=to_oracle(page), shared_gate_logits=None, routed_scaling_factor=1.0)
    else:
        with tiled_min_tokens(1 << 62):
            y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False,
                                          return_routing=True)
        torch.cuda.synchronize()
        y_ref, w_ref, ids_ref = _oracle_forward(x, logits, pool, slots, k, True)
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    parity(f32_of(y), y_ref, TOL[dtype], case=f"xcd order T={T} E={E} k={k} Is={Is}")
