"""The single-launch layer (layer1.hip) hands the activation rows from its gate/up workgroups to
its down workgroups inside one launch. This test compiles layer1.hip for gfx950 with the
library's own flags and checks the protocol in the compiled code of every instantiation:

  - no L2 write-back or invalidate instructions are needed or present (every hand-over goes
    through device-scope -- sc1 -- stores and loads);
  - publication: the last device-scope store of the program (the flag) follows a workgroup
    barrier, which follows a wait for all vector-memory operations, with no memory operation
    in between -- every activation store of every wave has completed before the flag is set;
  - the activation rows are stored with device-scope stores;
  - the poll: a loop whose body loads the flags with device-scope loads, all in flight at once,
    reads the wall clock and sleeps; its exit depends on the clock (a bounded wait);
  - after the poll and a barrier, the activation rows are read with device-scope loads.
Runs on the CPU: hipcc cross-compiles; no GPU is used.
"""
import os
import re
import shutil
import subprocess

import pytest

from ae_amd import build as libbuild

# gateup_kernel<..., FD = true, ST = false>: its last two template arguments
FD_RE = re.compile(r"^(_ZN3smx13gateup_kernel\w*Lb1ELb0EEEvNS_10ExpertArgsE):")


@pytest.fixture(scope="module")
def fd_kernels(tmp_path_factory):
    hipcc = next((c for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc") if c and os.path.exists(c)), None)
    if hipcc is None:
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("isa") / "layer1.s"
    src = os.path.join(libbuild.CSRC, "layer1.hip")
    proc = subprocess.run([hipcc, *libbuild.HIPCC_FLAGS, "--cuda-device-only", "-S", src, "-o", str(out)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    lines = out.read_text().split("\n")
    funcs = {}
    for i, line in enumerate(lines):
        m = FD_RE.match(line)
        if m:
            end = next(j for j in range(i, len(lines)) if lines[j].startswith(".Lfunc_end"))
            funcs[m.group(1)] = [l.split(";")[0].strip() for l in lines[i:end]]
    return funcs


def _is_vmem(t):
    op = t.split()[0] if t else ""
    return op.startswith(("global_", "buffer_", "flat_", "scratch_"))


def test_every_instantiation_found(fd_kernels):
    assert len(fd_kernels) == 12, sorted(fd_kernels)  # 3 dtypes x 4 top-k lane groups


def test_no_cache_maintenance(fd_kernels):
    for name, body in fd_kernels.items():
        assert not any(t.startswith(("buffer_wbl2", "buffer_inv")) for t in body), name


def test_publication_follows_completed_stores(fd_kernels):
    for name, body in fd_kernels.items():
        stores = [i for i, t in enumerate(body) if t.startswith("global_store") and t.endswith("sc1")]
        assert len(stores) >= 2, name  # activation stores and the flag
        flag = stores[-1]
        # walk back: no memory operation until the barrier, then a vmcnt(0) wait before it
        i = flag - 1
        while not body[i].startswith("s_barrier"):
            assert not _is_vmem(body[i]), (name, body[i])
            i -= 1
        # the wait is in the same straight-line block as the barrier (no label in between)
        j = i - 1
        while not (body[j].startswith("s_waitcnt") and "vmcnt(0)" in body[j]):
            assert not _is_vmem(body[j]), (name, body[j])
            assert not body[j].startswith(".LBB"), (name, "no vmcnt(0) before the publishing barrier")
            j -= 1


def test_poll_is_bounded_and_device_scope(fd_kernels):
    for name, body in fd_kernels.items():
        sleeps = [i for i, t in enumerate(body) if t.startswith("s_sleep")]
        assert len(sleeps) == 1, name
        s = sleeps[0]
        # the loop around the sleep: a backward branch after it to a label before it
        labels = {t[:-1]: i for i, t in enumerate(body) if t.startswith(".LBB") and t.endswith(":")}
        back = [(i, t.split()[-1]) for i, t in enumerate(body[s:], s)
                if t.startswith(("s_branch", "s_cbranch")) and labels.get(t.split()[-1], 1 << 30) < s]
        assert back, name
        head = min(labels[lbl] for _, lbl in back)
        loop = body[head:back[0][0] + 1]
        loads = [t for t in loop if t.startswith("global_load") and t.endswith("sc1")]
        assert len(loads) == 8, (name, loads)  # every flag load of a poll in flight together
        assert any(t.startswith("s_memrealtime") for t in loop), name
        first_wait = next(i for i, t in enumerate(loop) if t.startswith("s_waitcnt") and "vmcnt" in t)
        first_load = next(i for i, t in enumerate(loop) if t.startswith("global_load") and t.endswith("sc1"))
        assert all(not (t.startswith("global_load") and t.endswith("sc1")) for t in loop[first_wait:]), name
        assert first_load < first_wait, name


def test_activation_rows_read_at_device_scope_after_the_poll(fd_kernels):
    for name, body in fd_kernels.items():
        sleep = next(i for i, t in enumerate(body) if t.startswith("s_sleep"))
        reads = [i for i, t in enumerate(body) if t.startswith("buffer_load") and t.endswith("sc1")]
        assert len(reads) == 8, name  # a thread's staging loads, in flight together
        barrier = next(i for i in range(sleep, len(body)) if body[i].startswith("s_barrier"))
        assert all(i > barrier for i in reads), name
