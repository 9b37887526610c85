"""The oracle at full layer shapes, pinned against regression: on the deterministic inputs of
tests/golden/synth.py (C1 in fp32, the Mixtral-8x7B layer at one token, the DeepSeek-V2-Lite
and Qwen1.5-MoE blocks) the oracle must reproduce the committed output bits, routing weight
bits and ids exactly (written by tests/golden/make_oracle_fixtures.py)."""
import json
import os

import numpy as np
import pytest

from oracle import moe_ref as ref
from tests.golden.make_oracle_fixtures import MANIFEST, digest
from tests.golden.synth import CASES, bits_of, make_case, oracle_forward

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fixture(name):
    with np.load(os.path.join(HERE, f"oracle_{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_manifest_lists_every_case():
    with open(MANIFEST) as f:
        man = json.load(f)
    assert sorted(man) == sorted(CASES)
    for name, m in man.items():
        fx = _fixture(name)
        assert digest(fx["y_bits"]) == m["y_sha256"]
        assert digest(fx["w_bits"]) == m["w_sha256"]
        assert digest(fx["ids"]) == m["ids_sha256"]


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    case = make_case(name)
    y, w, ids = oracle_forward(case)
    fx = _fixture(name)
    np.testing.assert_array_equal(np.asarray(ids, np.int32), fx["ids"])
    np.testing.assert_array_equal(np.ascontiguousarray(w, np.float32).view(np.uint32), fx["w_bits"])
    np.testing.assert_array_equal(bits_of(y, case["dtype"]), fx["y_bits"])
    # the inputs the GPU tests upload route to the fixture's experts, and only their pages are set
    active = sorted(set(int(v) for v in fx["ids"].reshape(-1)))
    slots = case["slot_map"]
    head = ref.to_f32(case["pool"][:, :8], case["dtype"])
    filled = [p for p in range(case["P"]) if not np.isnan(head[p]).any()]
    assert sorted(int(slots[e]) for e in active) == filled
