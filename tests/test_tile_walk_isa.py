"""The 16-bit tiled kernels (tiles.hip) fill their token stages by LDS DMA and publish each
stage to the other waves with a plain workgroup barrier after a counted `s_waitcnt vmcnt(n)`.
The count is only right if the wave issued its vector-memory operations in the order the
source states (a step's token DMA, then its weight loads). This test compiles tiles.hip for
gfx950 with the library's own flags and checks that, in the compiled code, every barrier of the
K walk is preceded by a wait that retires the DMA group the next step reads:

  - the walk's first region (before the first barrier) issues DMA(0), W(0), DMA(1), W(1), and a
    wait in it leaves DMA(0) complete;
  - every later region issues DMA, then weights (4 + 8 operations), and a wait in it leaves the
    previous region's DMA group complete (also across the loop's back edge).

A compiler that issued the first weights ahead of the first DMA broke exactly this once (the
first DMA was still in flight at the barrier and other waves read stale LDS). Runs on the CPU:
hipcc cross-compiles; no GPU is used.
"""
import os
import re
import shutil
import subprocess

import pytest

from ae_amd import build as libbuild

KERNEL_RE = re.compile(r"^(_ZN3smx\d+tile_(gateup|down)_kernelILi([12])EEEvNS_10ExpertArgsE):")
DMA_GROUP = 4      # token DMA instructions per step and wave
W_GROUP = 8        # weight loads per step and wave


def _hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.fixture(scope="module")
def tile_asm(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("isa") / "tiles.s"
    src = os.path.join(libbuild.CSRC, "tiles.hip")
    cmd = [hipcc, *libbuild.HIPCC_FLAGS, "--cuda-device-only", "-S", src, "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return out.read_text().split("\n")


def _functions(lines):
    funcs = {}
    for i, line in enumerate(lines):
        m = KERNEL_RE.match(line)
        if m:
            end = next(j for j in range(i, len(lines)) if lines[j].startswith(".Lfunc_end"))
            funcs[m.group(1)] = lines[i:end]
    return funcs


def _events(body):
    """The walk's instruction stream as events: 'D' (buffer load into LDS), 'L' (other vector
    load), ('w', n) (s_waitcnt with a vmcnt field), 'B' (s_barrier)."""
    ev = []
    for line in body:
        t = line.split(";")[0].strip()
        if not t:
            continue
        op = t.split()[0]
        if op.startswith("buffer_load") or op.startswith("global_load"):
            ev.append("D" if t.endswith(" lds") else "L")
        elif op.startswith("buffer_store") or op.startswith("global_store"):
            ev.append("S")
        elif op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", t)
            if m:
                ev.append(("w", int(m.group(1))))
        elif op == "s_barrier":
            ev.append("B")
    return ev


def _regions(ev):
    regions, cur = [], []
    for e in ev:
        if e == "B":
            regions.append(cur)
            cur = []
        else:
            cur.append(e)
    regions.append(cur)
    return regions


def _vm_ops(region):
    return [e for e in region if e in ("D", "L", "S")]


def _retired_by_wait(region, ops_before_region_after_group, group_end_index=None):
    """True when some wait in `region` retires a DMA group. The group was followed by
    `ops_before_region_after_group` vector-memory operations before this region began; within
    the region, only waits after index `group_end_index` count (the group's own end, when the
    group is in this region)."""
    issued_after = ops_before_region_after_group
    for i, e in enumerate(region):
        if group_end_index is not None and i <= group_end_index:
            continue
        if e in ("D", "L", "S"):
            issued_after += 1
        elif isinstance(e, tuple) and e[1] <= issued_after:
            return True
    return False


def _ops_after_last_dma(region):
    vm = _vm_ops(region)
    last = max(i for i, e in enumerate(vm) if e == "D")
    return len(vm) - 1 - last


def test_all_16bit_tile_kernels_found(tile_asm):
    names = sorted(_functions(tile_asm))
    assert len(names) == 4, names  # gate/up and down, fp16 and bf16


def test_walk_waits_cover_each_dma_group(tile_asm):
    for name, body in _functions(tile_asm).items():
        regions = _regions(_events(body))
        walk = [i for i, r in enumerate(regions) if "D" in r]
        assert len(walk) >= 3, (name, walk)
        # the prologue: ... DMA(0) W(0) DMA(1) W(1), then waits
        pro = regions[walk[0]]
        vm = _vm_ops(pro)
        tail = "".join(vm[-2 * (DMA_GROUP + W_GROUP):])
        assert tail == ("D" * DMA_GROUP + "L" * W_GROUP) * 2, (name, "".join(vm))
        first_d = [i for i, e in enumerate(pro) if e == "D"][DMA_GROUP - 1]
        assert _retired_by_wait(pro, 0, first_d), (name, "prologue barrier passes with DMA(0) in flight")
        # every step of the walk: DMA then weights, and the previous region's DMA retired
        for a, b in zip(walk, walk[1:]):
            assert b == a + 1, (name, "a walk region without token DMA between barriers")
            seq = "".join(_vm_ops(regions[b]))
            assert seq == "D" * DMA_GROUP + "L" * W_GROUP, (name, b, seq)
            assert _retired_by_wait(regions[b], _ops_after_last_dma(regions[a])), (name, b)
        # the loop's back edge: the first step after the prologue also follows the last step
        first_step = regions[walk[1]]
        assert _retired_by_wait(first_step, _ops_after_last_dma(regions[walk[-1]])), name


def test_walk_ends_with_no_dma_in_flight(tile_asm):
    """After the last barrier no DMA is issued, and a vmcnt(0) wait follows the last one."""
    for name, body in _functions(tile_asm).items():
        ev = _events(body)
        last_d = max(i for i, e in enumerate(ev) if e == "D")
        assert "B" in ev[last_d:], name
        assert any(isinstance(e, tuple) and e[1] == 0 for e in ev[last_d:]), name
