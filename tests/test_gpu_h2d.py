"""GPU tests of the pinned host allocator and the host -> device transfer engine (expert page
streaming into pool slots), through the C ABI."""
import time

import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd import _lib
from ae_amd.backend import (HtoDTransferEngine, free_pinned_tensor, make_pinned_numpy_array,
                            make_pinned_tensor)
from ae_amd.layers import fused_moe_forward
from tests.helpers import TOL, TORCH_TO_ORACLE, f32_of, max_rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pinned_tensor_round_trip(dtype):
    torch.zeros(1, device=DEV)  # torch reports pinned memory once its device context exists
    t, p = make_pinned_tensor(1 << 20, dtype)
    try:
        assert t.dtype == dtype and t.numel() == (1 << 20) // t.element_size()
        assert t.is_pinned()
        src = torch.randn(t.numel()).to(dtype)
        t.copy_(src)
        g = t.to(DEV, non_blocking=True)
        torch.cuda.synchronize()
        assert torch.equal(g.cpu(), src)
    finally:
        free_pinned_tensor(p)


def test_pinned_numpy_view():
    t, p = make_pinned_tensor(4096, torch.float32)
    try:
        a = make_pinned_numpy_array(p, 1024, np.float32)
        a[:] = np.arange(1024, dtype=np.float32)
        assert torch.equal(t, torch.arange(1024, dtype=torch.float32))
    finally:
        free_pinned_tensor(p)


@pytest.mark.parametrize("num_chunks", [1, 3, 7])
def test_weight_pages_stream_into_slots(num_chunks):
    """Expert pages from a pinned host copy of the layer's experts into non-contiguous pool
    slots, one task per page, bit-exact (bf16)."""
    E, page = 4, 3 * 256 * 384 + 5  # odd element count: uneven chunks
    host, p = make_pinned_tensor(E * page * 2, torch.bfloat16)
    try:
        host = host.view(E, page)
        host.copy_(torch.randn((E, page)).to(torch.bfloat16))
        pool = torch.zeros((8, page), dtype=torch.bfloat16, device=DEV)
        slots = [0, 2, 3, 6]
        eng = HtoDTransferEngine()
        eng.start()
        stream = torch.cuda.Stream()
        for e, s in enumerate(slots):
            eng.submit_weight_loading_task(host[e], pool[s], stream, f"w{e}", num_chunks, layer_id=1)
        for e in range(E):
            ok, secs = eng.wait_for_completion(f"w{e}", timeout=30.0)
            assert ok and secs is not None and secs >= 0.0
        for e, s in enumerate(slots):
            assert torch.equal(pool[s].cpu(), host[e])
        for s in (1, 4, 5, 7):
            assert int(pool[s].abs().sum().item()) == 0
        eng.clear_condition([f"w{e}" for e in range(E)])
        assert not eng.has_task_id("w0")
        eng.stop()
    finally:
        free_pinned_tensor(p)


def test_priority_order_and_timeouts():
    """Paused worker, three queued tasks: the draft-KV task runs first, then weight layer 1,
    then weight layer 2 (each a 96 MiB copy, long enough that the next one cannot have finished
    when the previous one is reported)."""
    n = 96 << 20
    host, p = make_pinned_tensor(3 * n, torch.float16)
    try:
        host = host.view(3, -1)
        host.fill_(1.0)
        dst = torch.empty((3, host.shape[1]), dtype=torch.float16, device=DEV)
        eng = HtoDTransferEngine()
        eng.start()
        stream = torch.cuda.Stream()
        eng.set_worker_enabled(False)
        eng.submit_weight_loading_task(host[0], dst[0], stream, "w2", 1, layer_id=2)
        eng.submit_weight_loading_task(host[1], dst[1], stream, "w1", 1, layer_id=1)
        eng.submit_draft_kv_cache_loading_task(host[2], dst[2], stream, "kv", 1)
        assert eng.pending_chunks() == 3
        assert eng.wait_for_completion("kv", timeout=0.05) is False   # paused: times out
        eng.set_worker_enabled(True)
        assert eng.wait_for_completion("kv", timeout=30.0) is True
        assert eng.wait_for_completion("w1", timeout=0.0) is False  # still running
        assert eng.wait_for_completion("w1", timeout=30.0)[0] is True
        assert eng.wait_for_completion("w2", timeout=0.0) is False
        assert eng.wait_for_completion("w2", timeout=30.0)[0] is True
        torch.cuda.synchronize()
        assert bool((dst == 1.0).all())
        assert eng.wait_for_completion("nope") is False
        eng.stop()
    finally:
        free_pinned_tensor(p)


def test_streamed_pages_feed_the_moe_forward():
    """Experts streamed from pinned host memory by the engine into a slot map, then the fused
    forward reads them: same result as the oracle on the host pages."""
    T, H, I, E, k = 12, 256, 256, 4, 2
    page = 3 * I * H
    host, p = make_pinned_tensor(E * page * 2, torch.bfloat16)
    try:
        host = host.view(E, page)
        host.copy_((torch.randn((E, page)) * 0.02).to(torch.bfloat16))
        pool = torch.full((2 * E, page), float("nan"), dtype=torch.bfloat16, device=DEV)
        slots = torch.tensor([1, 3, 5, 7], dtype=torch.int64, device=DEV)
        eng = HtoDTransferEngine()
        eng.start()
        stream = torch.cuda.Stream()
        for e in range(E):
            eng.submit_weight_loading_task(host[e], pool[int(slots[e])], stream, f"p{e}", 2, layer_id=3)
        for e in range(E):
            assert eng.wait_for_completion(f"p{e}", timeout=30.0)[0]
        eng.stop()
        g = torch.Generator(device=DEV).manual_seed(1)
        x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
        logits = (torch.randn((T, E), generator=g, device=DEV) * 2).to(torch.bfloat16)
        y = fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)
        torch.cuda.synchronize()
        host_pool = np.zeros((2 * E, page), np.uint16)
        host_pool[slots.cpu().numpy()] = to_oracle(host)
        y_ref, _, _ = ref.fused_moe_forward(to_oracle(x), f32_of(logits), host_pool,
                                            slots.cpu().numpy(), k, True, ref.BF16)
        assert max_rel_err(f32_of(y), y_ref) <= TOL[torch.bfloat16]
    finally:
        free_pinned_tensor(p)
