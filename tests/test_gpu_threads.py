"""Calls from several host threads, each on its own stream with its own workspace, give the bits
of the same calls made one at a time -- the C ABI's contract (stream-ordered, no host
synchronisation, re-entrant for distinct workspaces), which the reference relies on when its
attention executor thread and the main thread launch on the GPU (execution_engine.py:855)."""
import threading

import pytest
import torch

from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward
from tests.helpers import make_pool

pytestmark = pytest.mark.gpu
DEV = "cuda"

# T, H, I, E, k, shared I: one-wave routing, in-launch routing, the routing kernels and the
# MFMA-tiled kernels (600 tokens x top-2 over 8 experts), and a shared-expert block
CASES = [(1, 256, 128, 8, 2, 0), (24, 256, 256, 16, 4, 0), (130, 128, 256, 8, 2, 0),
         (600, 256, 256, 8, 2, 0), (33, 256, 128, 16, 4, 256)]


def _inputs(case, seed):
    T, H, I, E, k, Is = case
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = (torch.randn((T, E), generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    pool, slots = make_pool(E, H, I, torch.bfloat16, num_slots=E + 1, seed=seed + 1)
    page = (torch.randn((3 * Is * H,), generator=g, device=DEV) * 0.02).to(torch.bfloat16) if Is else None
    return x, logits, pool, slots, page


def _call(case, inp):
    T, H, I, E, k, Is = case
    x, logits, pool, slots, page = inp
    if Is:
        return fused_moe_shared_forward(x.clone(), logits, pool, slots, k, False, page, None, 1.5,
                                        inplace=False)
    return fused_moe_forward(x.clone(), logits, pool, slots, k, True, inplace=False)


def test_threads_on_their_own_streams_match_serial_calls():
    inputs = [_inputs(c, seed=100 + i) for i, c in enumerate(CASES)]
    torch.cuda.synchronize()
    want = [_call(c, inp) for c, inp in zip(CASES, inputs)]
    torch.cuda.synchronize()
    got = [[] for _ in CASES]
    errors = []

    def work(i):
        try:
            s = torch.cuda.Stream()  # default priority
            with torch.cuda.stream(s):
                for _ in range(6):
                    got[i].append(_call(CASES[i], inputs[i]))
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(CASES))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i, case in enumerate(CASES):
        assert len(got[i]) == 6, case
        for y in got[i]:
            assert torch.equal(y, want[i]), case
