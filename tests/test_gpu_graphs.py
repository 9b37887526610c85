"""Every entry point captured in a HIP graph (torch.cuda.graph): each replay, with eager calls
of the same entry point and host synchronisations between replays, gives the eager result bit
for bit. Covers the forms the shared-expert graph test does not: the whole post-attention
layer call (in place, inputs restored inside the graph), caller routing, the grouped top-k and
the block on its routing, the MFMA-tiled kernels and the allocation-free entry point. The
library records no memset and no host synchronisation, so every call is capturable."""
import pytest
import torch

from ae_amd import _lib
from ae_amd.layers import (fused_moe_forward, grouped_topk, moe_layer_forward, stack_fused_moe,
                           stack_fused_moe_shared, tiled_min_tokens)
from ae_amd.layers._torch import dtype_code, ptr, stream_of
from tests.helpers import make_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _replays_match(run, out):
    """Capture out.copy_(run()) after a warm-up on a side stream; replay 4 times against the
    eager result, with eager runs between the replays."""
    eager = run().clone()
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
        run()
        torch.cuda.synchronize()


def _inputs(T, H, E, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(BF)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(BF)
    return x, logits, g


@pytest.mark.parametrize("T", [1, 24])
def test_layer_call_graph(T):
    H, I, E, k, Is = 256, 128, 16, 4, 256
    x, _, g = _inputs(T, H, E, seed=10 + T)
    res = torch.randn((T, H), generator=g, device=DEV).to(BF)
    nw = (1.0 + 0.1 * torch.randn((H,), generator=g, device=DEV)).to(BF)
    gw = (torch.randn((E, H), generator=g, device=DEV) * 0.05).to(BF)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(BF)
    pool, slots = make_pool(E, H, I, BF, num_slots=E + 1, seed=11 + T)
    h, r = torch.empty_like(x), torch.empty_like(res)
    out = torch.empty((T, 2 * H), device=DEV, dtype=BF)

    def run():
        h.copy_(x)
        r.copy_(res)
        moe_layer_forward(h, r, nw, 1e-6, gw, pool, slots, k, False, shared_w=page,
                          routed_scaling_factor=2.0)
        return torch.cat([h, r], dim=1)

    _replays_match(run, out)


def test_caller_routing_graph():
    T, H, I, E, k = 40, 256, 128, 16, 3
    x, logits, g = _inputs(T, H, E, seed=20)
    pool, slots = make_pool(E, H, I, BF, seed=21)
    ids = torch.stack([torch.randperm(E, generator=torch.Generator().manual_seed(t))[:k]
                       for t in range(T)]).to(device=DEV, dtype=torch.int32)
    w = torch.rand((T, k), generator=g, device=DEV)
    out = torch.empty_like(x)
    _replays_match(lambda: stack_fused_moe(x, pool, slots, logits, w, ids, False, inplace=False), out)


@pytest.mark.parametrize("biased", [False, True])
def test_grouped_routing_block_graph(biased):
    T, H, I, E, k, Is = 12, 256, 128, 32, 6, 256
    x, logits, g = _inputs(T, H, E, seed=30 + int(biased))
    pool, slots = make_pool(E, H, I, BF, seed=31)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(BF)
    bias = torch.randn((E,), generator=g, device=DEV) * 0.1 if biased else None
    out = torch.empty_like(x)

    def run():
        w, ids = grouped_topk(logits, k, biased, 8, 3, bias)
        return stack_fused_moe_shared(x, pool, slots, w, ids, page, None, 2.5, inplace=False)

    _replays_match(run, out)


def test_tiled_kernels_graph():
    T, H, I, E, k = 1024, 256, 256, 8, 2
    x, logits, _ = _inputs(T, H, E, seed=40)
    pool, slots = make_pool(E, H, I, BF, seed=41)
    out = torch.empty_like(x)
    with tiled_min_tokens(0):
        assert _lib.plan_info(T, H, I, E, k, _lib.SMX_BF16)["tiled"] == 1
        _replays_match(lambda: fused_moe_forward(x, logits, pool, slots, k, True, inplace=False), out)


def test_noalloc_entry_point_graph():
    T, H, I, E, k = 16, 256, 128, 8, 2
    x, logits, _ = _inputs(T, H, E, seed=50)
    pool, slots = make_pool(E, H, I, BF, seed=51)
    y = torch.empty_like(x)
    w = torch.empty((T, k), dtype=torch.float32, device=DEV)
    ids = torch.empty((T, k), dtype=torch.int32, device=DEV)
    out = torch.empty_like(x)

    def run():
        _lib.call("smx_fused_moe_forward_noalloc", ptr(x), ptr(y), dtype_code(BF), T, H, ptr(logits),
                  dtype_code(BF), E, k, 1, ptr(pool), pool.shape[0], pool.shape[1], ptr(slots),
                  ptr(w), ptr(ids), stream_of(x))
        return y

    _replays_match(run, out)
