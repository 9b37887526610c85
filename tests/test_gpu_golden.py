"""The GPU path against the committed oracle fixtures at full layer shapes (C1 in fp32 through
a slot map, the Mixtral-8x7B layer at one token, the DeepSeek-V2-Lite and Qwen1.5-MoE blocks),
on the deterministic inputs of tests/golden/synth.py: ids and routing weight bits exact,
outputs within the parity tolerance. Unrouted pool pages hold NaN, so a read of one shows."""
import os

import numpy as np
import pytest
import torch

from ae_amd.layers import fused_moe_forward, fused_moe_shared_forward
from oracle import moe_ref as ref
from tests.golden.synth import CASES, make_case
from tests.helpers import TOL_BY_NAME, f32_of, parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _dev(a, dtype):
    """Storage array (bf16 bit patterns, or fp32) -> device tensor of the activation dtype."""
    a = np.ascontiguousarray(a)
    if dtype == "bf16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a).to(DEV)


@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_matches_oracle_fixture(name):
    case = make_case(name)
    dt = case["dtype"]
    x = _dev(case["x"], dt)
    logits = torch.from_numpy(case["logits"]).to(_DT[dt]).to(DEV)  # values exact in dt
    pool = _dev(case["pool"], dt)
    slots = torch.from_numpy(case["slot_map"]).to(DEV)
    if case["Is"]:
        page = _dev(case["shared_page"], dt)
        sg = None if case["shared_gate"] is None else torch.from_numpy(case["shared_gate"]).to(_DT[dt]).to(DEV)
        y, w, ids = fused_moe_shared_forward(x.clone(), logits, pool, slots, case["k"], case["renorm"],
                                             page, sg, 1.0, inplace=False, return_routing=True)
    else:
        y, w, ids = fused_moe_forward(x.clone(), logits, pool, slots, case["k"], case["renorm"],
                                      inplace=False, return_routing=True)
    torch.cuda.synchronize()
    with np.load(os.path.join(HERE, f"oracle_{name}.npz"), allow_pickle=False) as z:
        want_y, want_w, want_ids = z["y_bits"], z["w_bits"], z["ids"]
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), want_w)
    y_ref = ref.bf16_bits_to_f32(want_y) if dt == "bf16" else want_y.view(np.float32)
    parity(f32_of(y), y_ref, TOL_BY_NAME[dt], case=f"golden {name}")
