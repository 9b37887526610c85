"""Write the oracle fixtures of the full-size layer cases (tests/golden/synth.py):
oracle_<case>.npz with the output bits, routing weight bits and ids of each case, and
oracle_fixtures.json with their sha256 digests. Run from the repository root:

    python -m tests.golden.make_oracle_fixtures

tests/test_golden_fixtures.py re-runs the oracle on the same inputs and requires these bits;
tests/test_gpu_golden.py checks the GPU path against them.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

from tests.golden.synth import CASES, bits_of, make_case, oracle_forward

HERE = os.path.dirname(os.path.abspath(__file__))
MANIFEST = os.path.join(HERE, "oracle_fixtures.json")


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    manifest = {}
    for name in CASES:
        case = make_case(name)
        y, w, ids = oracle_forward(case)
        yb = bits_of(y, case["dtype"])
        wb = np.ascontiguousarray(w, np.float32).view(np.uint32)
        ids = np.ascontiguousarray(ids, np.int32)
        np.savez_compressed(os.path.join(HERE, f"oracle_{name}.npz"), y_bits=yb, w_bits=wb, ids=ids)
        manifest[name] = {
            "shape": {k: case[k] for k in ("T", "H", "I", "E", "k", "Is", "P")},
            "dtype": case["dtype"],
            "active_experts": sorted(set(int(v) for v in ids.reshape(-1))),
            "y_sha256": digest(yb),
            "w_sha256": digest(wb),
            "ids_sha256": digest(ids),
            "max_abs_y": float(np.abs(y).max()),
        }
        print(name, manifest[name]["active_experts"], manifest[name]["y_sha256"][:16], flush=True)
    with open(MANIFEST, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
