"""The expert-ordered gate/up items (gateup_kernel with ST) issue their first item's weight loads
before routing the batch, so that the routing runs while the weights are in flight. That holds
only if the compiled code keeps them in flight: vector loads complete in issue order, so a
wait for any load issued after them waits for them too. This test compiles one instantiation
(bf16, two token tiles, 64 lanes per token, the K split between wave pairs) for gfx950 with the
library's flags and checks in its code:
  - no scratch memory (the prefetched registers must not spill);
  - the routing's own loads (caller ids, the expert-to-slot map) are issued before the 16
    weight loads (non-temporal buffer loads of two chunks x 4 instructions x 2 tiles);
  - the routing's waits for its own loads (before it copies the caller ids and the slots into
    LDS, and in the sort) leave those 16 loads outstanding;
  - the item's range record is read from LDS (no flat loads, which would count as vector
    loads and wait for the weights).
Runs on the CPU: hipcc cross-compiles; no GPU is used.
"""
import os
import re
import shutil
import subprocess

import pytest

from ae_amd import build as libbuild

TU = """
#include "{csrc}/gateup_device.h"
namespace smx {{
template __global__ void gateup_kernel<false, kBF16, 2, 64, true, 4, false, true, false, true>(ExpertArgs);
}}
"""


@pytest.fixture(scope="module")
def body(tmp_path_factory):
    hipcc = next((c for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc") if c and os.path.exists(c)), None)
    if hipcc is None:
        pytest.skip("hipcc is not installed")
    d = tmp_path_factory.mktemp("prefetch")
    src = d / "one.hip"
    src.write_text(TU.format(csrc=libbuild.CSRC))
    out = d / "one.s"
    proc = subprocess.run([hipcc, *libbuild.HIPCC_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return [l.split(";")[0].strip() for l in out.read_text().split("\n")]


def _vmcnt(t):
    m = re.search(r"vmcnt\((\d+)\)", t)
    return int(m.group(1)) if m else None


def test_no_scratch(body):
    sizes = [int(t.split()[-1]) for t in body if t.startswith(".amdhsa_private_segment_fixed_size")]
    assert sizes == [0], sizes


def test_routing_loads_before_weights(body):
    weights = [i for i, t in enumerate(body) if t.startswith("buffer_load_dwordx4") and t.endswith(" nt")]
    assert len(weights) >= 16
    first_w = weights[0]
    assert weights[15] - first_w < 80, "the 16 weight loads are issued together"
    routing = [i for i, t in enumerate(body[:first_w]) if t.startswith("global_load")]
    assert len(routing) >= 2, "caller ids and the expert-to-slot map are loaded first"


def _last_wait(body, i, span=16):
    waits = [_vmcnt(t) for t in body[max(0, i - span):i] if _vmcnt(t) is not None]
    return waits[-1] if waits else None


def test_routing_waits_leave_weights_in_flight(body):
    weights = [i for i, t in enumerate(body) if t.startswith("buffer_load_dwordx4") and t.endswith(" nt")]
    last_w = weights[15]
    # the caller ids' LDS copy (ids outside [0, E) become -2) and then the slots' copy: the waits
    # before them leave the 16 weight loads outstanding
    ids_w = next(i for i in range(last_w, len(body)) if body[i].startswith("ds_write_b16") and
                 any("cndmask" in t and "-2" in t for t in body[i - 12:i]))
    assert _last_wait(body, ids_w) == 16, body[ids_w - 12:ids_w + 1]
    slot_w = next(i for i in range(ids_w, len(body)) if body[i].startswith("ds_write_b64"))
    assert _last_wait(body, slot_w, 30) == 16, body[slot_w - 30:slot_w + 1]
    # and the sort's waits (for its LDS work only) after them
    later = [_vmcnt(t) for t in body[slot_w:slot_w + 1200] if _vmcnt(t) is not None]
    assert later.count(16) >= 4, later[:20]


def test_no_flat_loads(body):
    assert not any(t.startswith("flat_load") for t in body)
