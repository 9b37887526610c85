"""CPU checks of the C ABI: the library loads, exports exactly what include/specmoe_mi355x.h
declares, and rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

from ae_amd import _lib
from ae_amd.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "specmoe_mi355x.h")
L = _lib.lib()
VP = ctypes.c_void_p
A = VP(0x10000)  # an aligned fake address: the calls below return before dereferencing it


def _declared():
    with open(HEADER) as f:
        text = f.read()
    return re.findall(r"^\s*(?:int64_t|int|size_t|const char\*)\s+(smx_\w+)\s*\(", text, re.M)


def test_library_built_in_tree():
    assert os.path.exists(LIB_PATH)
    assert os.path.dirname(LIB_PATH).endswith("ae_amd")


def test_exports_every_declared_symbol():
    names = _declared()
    assert len(names) == 45, names
    assert sorted(names) == sorted(n for n, _, _ in _lib.SIGNATURES)
    for n in names:
        assert hasattr(L, n), n


def test_one_hip_runtime_when_loaded_before_torch():
    """Loading the library first must not leave two HIP runtimes mapped in the process."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); from ae_amd import _lib; _lib.lib(); import torch; "
            "maps = open('/proc/self/maps').read().splitlines(); "
            "print(len({l.split()[-1] for l in maps if 'libamdhip64' in l}))" % root)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "1", out.stdout


def test_version_and_error_strings():
    assert L.smx_version() == 10100
    for code, word in [(0, b"success"), (1000, b"invalid"), (1001, b"supported"),
                       (1002, b"workspace"), (1003, b"aligned")]:
        assert word in L.smx_error_string(code)


def test_plan_info_host_query():
    """smx_moe_plan_info runs on the host only: it answers here, without a GPU."""
    p = _lib.plan_info(32, 4096, 14336, 8, 2, _lib.SMX_BF16)
    assert p["tiled"] == 0 and p["span"] == 32 and p["max_ranges"] == 8 + 64 // 32
    assert p["workspace_bytes"] == L.smx_moe_workspace_size(32, 4096, 14336, 8, 2, 2)
    q = _lib.plan_info(256, 4096, 14336, 8, 2, _lib.SMX_BF16)
    assert q["tiled"] == 1 and q["span"] == 128 and q["tile_gateup_grid"] == q["max_ranges"] * 112
    s = _lib.plan_info(64, 2048, 1408, 64, 6, _lib.SMX_BF16, 2816)
    assert s["shared_tok_groups"] == 1 and s["shared_gateup_blocks"] > 0
    out = (ctypes.c_int64 * 2)()
    assert L.smx_moe_plan_info(32, 4096, 14336, 8, 2, 0, 2, out, 2) == len(_lib.PLAN_FIELDS)
    assert L.smx_moe_plan_info(32, 4096, 14336, 8, 9, 0, 2, out, 2) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_moe_plan_info(32, 4000, 14336, 8, 2, 0, 2, out, 2) == _lib.SMX_ERR_UNSUPPORTED
    assert L.smx_moe_plan_info(32, 4096, 14336, 8, 2, 0, 2, None, 2) == _lib.SMX_ERR_INVALID_ARG


def test_workspace_size():
    ws = L.smx_moe_workspace_size
    assert ws(32, 4096, 14336, 8, 2, 2) > 0
    assert ws(64, 4096, 14336, 8, 2, 2) > ws(32, 4096, 14336, 8, 2, 2)
    assert ws(32, 4096, 14336, 8, 2, 0) > ws(32, 4096, 14336, 8, 2, 2)  # fp32 intermediates
    assert ws(0, 4096, 14336, 8, 2, 2) > 0
    # rejected shapes report 0
    assert ws(32, 4000, 14336, 8, 2, 2) == 0   # H not a multiple of 128 (16-bit)
    assert ws(32, 4096, 14336, 300, 2, 2) == 0  # E > 256
    assert ws(32, 4096, 14336, 8, 9, 2) == 0    # top_k > E
    # more than 16384 assignments: token chunks of 8192 (top-2) share the workspace
    assert ws(9000, 4096, 14336, 8, 2, 2) == max(ws(8192, 4096, 14336, 8, 2, 2), ws(808, 4096, 14336, 8, 2, 2))
    assert ws(3000, 2048, 1408, 64, 6, 2) == max(ws(2730, 2048, 1408, 64, 6, 2), ws(270, 2048, 1408, 64, 6, 2))
    assert ws(32, 4096, 14336, 8, 2, 7) == 0    # bad dtype


def _stack(**kw):
    a = dict(hidden=A, out=A, dtype=2, T=4, H=256, pool=A, slots=4, page=3 * 256 * 256, e2s=A,
             E=4, w=A, ids=A, k=2, ws=A, wsb=1 << 30, stream=VP(0))
    a.update(kw)
    return L.smx_stack_fused_moe(a["hidden"], a["out"], a["dtype"], a["T"], a["H"], a["pool"],
                                 a["slots"], a["page"], a["e2s"], a["E"], a["w"], a["ids"],
                                 a["k"], a["ws"], a["wsb"], a["stream"])


def test_stack_rejects_before_launch():
    assert _stack(hidden=VP(0)) == _lib.SMX_ERR_INVALID_ARG
    assert _stack(page=1000) == _lib.SMX_ERR_INVALID_ARG           # not 3*I*H
    assert _stack(hidden=VP(0x10008)) == _lib.SMX_ERR_MISALIGNED
    assert _stack(k=5) == _lib.SMX_ERR_INVALID_ARG                 # top_k > E
    assert _stack(wsb=16) == _lib.SMX_ERR_WORKSPACE
    assert _stack(ws=VP(0x10004)) == _lib.SMX_ERR_MISALIGNED
    assert _stack(H=100, page=3 * 100 * 256) == _lib.SMX_ERR_UNSUPPORTED
    assert _stack(T=0) == _lib.SMX_OK                              # empty: nothing launched
    assert _stack(T=0, hidden=VP(0), out=VP(0), ws=VP(0)) == _lib.SMX_OK  # null data is fine
    assert _stack(T=-1) == _lib.SMX_ERR_INVALID_ARG


def test_stack_shared_rejects_before_launch():
    f = L.smx_stack_fused_moe_shared
    F = ctypes.c_float

    def call(**kw):
        a = dict(T=4, Is=256, page=A, sgate=VP(0), scale=F(1.0), wsb=1 << 30, k=2)
        a.update(kw)
        return f(A, A, 2, a["T"], 256, A, 4, 3 * 256 * 256, A, 4, A, A, a["k"], a["page"], a["Is"],
                 a["sgate"], a["scale"], A, a["wsb"], VP(0))
    assert call(T=0) == _lib.SMX_OK
    assert call(Is=-1) == _lib.SMX_ERR_INVALID_ARG
    assert call(Is=0) == _lib.SMX_ERR_INVALID_ARG                  # a page without a size
    assert call(Is=0, page=VP(0), sgate=A) == _lib.SMX_ERR_INVALID_ARG  # a gate without an expert
    assert call(scale=F(float("nan"))) == _lib.SMX_ERR_INVALID_ARG
    assert call(page=VP(0x10008)) == _lib.SMX_ERR_MISALIGNED
    assert call(k=5) == _lib.SMX_ERR_INVALID_ARG                   # top_k > E
    assert call(Is=100) == _lib.SMX_ERR_UNSUPPORTED                # shared I not a multiple of 128
    assert call(wsb=16) == _lib.SMX_ERR_WORKSPACE


def test_forward_and_routing_reject_before_launch():
    f = L.smx_fused_moe_forward
    args = [A, A, 2, 4, 256, A, 2, 4, 2, 1, A, 4, 3 * 256 * 256, A, VP(0), VP(0), A, 1 << 30, VP(0)]
    bad_logits = list(args)
    bad_logits[6] = 5
    assert f(*bad_logits) == _lib.SMX_ERR_INVALID_ARG
    zero = list(args)
    zero[3] = 0
    assert f(*zero) == _lib.SMX_OK
    assert L.smx_topk_softmax(A, 2, 0, 8, 2, 1, A, A, VP(0)) == _lib.SMX_OK
    assert L.smx_topk_softmax(A, 2, 4, 8, 9, 1, A, A, VP(0)) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_topk_softmax(A, 2, 4, 300, 2, 1, A, A, VP(0)) == _lib.SMX_ERR_UNSUPPORTED
    assert L.smx_moe_align_block_size(A, 10, 0, 16, A, A, A, VP(0)) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_moe_align_block_size(A, 20000, 8, 16, A, A, A, VP(0)) == _lib.SMX_ERR_UNSUPPORTED


def test_grouped_topk_rejects_before_launch():
    g = L.smx_grouped_topk
    ok, bad, uns = _lib.SMX_OK, _lib.SMX_ERR_INVALID_ARG, _lib.SMX_ERR_UNSUPPORTED
    # (T, E, k, groups, selected groups, bias) -> status
    cases = [((0, 160, 6, 8, 3, None), ok),
             ((4, 12, 1, 5, 1, None), bad),      # E not a multiple of the groups
             ((4, 12, 1, 4, 5, None), bad),      # more selected groups than groups
             ((4, 12, 1, 4, 0, None), bad),
             ((4, 12, 4, 4, 1, None), bad),      # k above the selectable experts (3)
             ((4, 12, 1, 12, 3, A), bad),        # a biased group score needs 2 experts a group
             ((4, 12, 0, 4, 1, None), bad),
             ((-1, 12, 1, 4, 1, None), bad),
             ((4, 300, 2, 1, 1, None), uns),     # E > 256
             ((4, 256, 1, 128, 1, None), uns),   # more groups than lanes
             ((4, 256, 17, 1, 1, None), uns)]    # k > 16
    for (T, E, k, ng, tg, bias), want in cases:
        assert g(A, 2, T, E, k, 1, ng, tg, bias, A, A, VP(0)) == want, (T, E, k, ng, tg)
    assert g(A, 7, 4, 160, 6, 1, 8, 3, None, A, A, VP(0)) == bad      # logits dtype
    assert g(None, 2, 4, 160, 6, 1, 8, 3, None, A, A, VP(0)) == bad   # no logits
    assert g(A, 2, 4, 160, 6, 1, 8, 3, None, None, A, VP(0)) == bad   # no weights out


def test_noalloc_forward_rejects_before_touching_the_device():
    """The no-allocation forward checks its arguments and its scratch bound before it looks up
    the device's scratch (no GPU here), and names the scratch in its error."""
    f = L.smx_fused_moe_forward_noalloc
    args = [A, A, 2, 4, 256, A, 2, 4, 2, 1, A, 4, 3 * 256 * 256, A, VP(0), VP(0), VP(0)]
    zero = list(args)
    zero[3] = 0
    assert f(*zero) == _lib.SMX_OK
    bad = list(args)
    bad[12] = 1000                                    # page not 3*I*H
    assert f(*bad) == _lib.SMX_ERR_INVALID_ARG
    bad = list(args)
    bad[8] = 5                                        # top_k > E
    assert f(*bad) == _lib.SMX_ERR_INVALID_ARG
    # Mixtral shape: 128 tokens fit the 32 MiB scratch, 256 do not
    big = [A, A, 2, 256, 4096, A, 2, 8, 2, 1, A, 8, 3 * 4096 * 14336, A, VP(0), VP(0), VP(0)]
    assert L.smx_moe_workspace_size(128, 4096, 14336, 8, 2, 2) <= _lib.SMX_NOALLOC_SCRATCH_BYTES
    assert L.smx_moe_workspace_size(256, 4096, 14336, 8, 2, 2) > _lib.SMX_NOALLOC_SCRATCH_BYTES
    assert f(*big) == _lib.SMX_ERR_SCRATCH
    assert b"scratch" in L.smx_error_string(_lib.SMX_ERR_SCRATCH)


def test_profile_events_argument_checks():
    assert L.smx_set_profile_events(None, 0) == _lib.SMX_OK
    three = (VP * 3)(A, A, A)
    assert L.smx_set_profile_events(three, 3) == _lib.SMX_ERR_INVALID_ARG
    holes = (VP * 5)(A, A, VP(0), A, A)
    assert L.smx_set_profile_events(holes, 5) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_set_profile_events(None, 0) == _lib.SMX_OK


def test_tiled_threshold_setting():
    """The tiled-kernel threshold is process-wide; the workspace query follows it (the tiled
    plan takes 128-token ranges and its own down-projection split)."""
    default = L.smx_tiled_min_tokens()
    assert default == 64
    try:
        never = (1 << 63) - 1
        assert L.smx_set_tiled_min_tokens(never) == _lib.SMX_OK
        assert L.smx_tiled_min_tokens() == never
        stream_ws = L.smx_moe_workspace_size(1024, 4096, 14336, 8, 2, 2)
        assert L.smx_set_tiled_min_tokens(0) == _lib.SMX_OK
        tiled_ws = L.smx_moe_workspace_size(1024, 4096, 14336, 8, 2, 2)
        assert tiled_ws > 0 and stream_ws > 0 and tiled_ws != stream_ws
    finally:
        assert L.smx_set_tiled_min_tokens(-1) == _lib.SMX_OK
    assert L.smx_tiled_min_tokens() == default


def test_fused_down_setting():
    """The fused down + combine setting is process-wide: negative = the default rule (at most
    48 KB of weight rows per output row), 0 = never, n = batches up to n tokens (capped at 8).
    Its plan needs no fp32 partials, so the workspace shrinks for batches it takes."""
    assert L.smx_fused_down_max_tokens() == -1
    ws = L.smx_moe_workspace_size
    sws = L.smx_moe_shared_workspace_size
    try:
        # default rule: DeepSeek-V2-Lite block at one token (23 units) fused, Mixtral (56) not
        ds_default = sws(1, 2048, 1408, 64, 6, 2816, 2)
        mx_default = ws(1, 4096, 14336, 8, 2, 2)
        assert L.smx_set_fused_down_max_tokens(0) == _lib.SMX_OK
        assert L.smx_fused_down_max_tokens() == 0
        assert sws(1, 2048, 1408, 64, 6, 2816, 2) > ds_default
        assert ws(1, 4096, 14336, 8, 2, 2) == mx_default
        split4 = ws(4, 4096, 14336, 8, 2, 2)
        assert L.smx_set_fused_down_max_tokens(100) == _lib.SMX_OK
        assert L.smx_fused_down_max_tokens() == 8
        assert 0 < ws(4, 4096, 14336, 8, 2, 2) < split4
        assert ws(1, 4096, 14336, 8, 2, 2) < mx_default
        # beyond 8 tokens the plan is the split one
        assert ws(9, 4096, 14336, 8, 2, 2) > ws(8, 4096, 14336, 8, 2, 2)
    finally:
        assert L.smx_set_fused_down_max_tokens(-1) == _lib.SMX_OK
    assert L.smx_fused_down_max_tokens() == -1


def test_fp32_gemm_outputs_fp16_setting():
    assert L.smx_fp32_gemm_outputs_fp16() == 0
    try:
        assert L.smx_set_fp32_gemm_outputs_fp16(1) == _lib.SMX_OK
        assert L.smx_fp32_gemm_outputs_fp16() == 1
        # it changes rounding only: the plans and workspace sizes stay the same
        assert L.smx_moe_workspace_size(32, 1024, 2816, 8, 2, 0) > 0
    finally:
        assert L.smx_set_fp32_gemm_outputs_fp16(0) == _lib.SMX_OK
    assert L.smx_fp32_gemm_outputs_fp16() == 0


def test_routing_in_gateup_setting():
    assert L.smx_routing_in_gateup() == 1
    try:
        assert L.smx_set_routing_in_gateup(0) == _lib.SMX_OK
        assert L.smx_routing_in_gateup() == 0
    finally:
        assert L.smx_set_routing_in_gateup(1) == _lib.SMX_OK
    assert L.smx_routing_in_gateup() == 1


def test_python_error_mapping():
    with pytest.raises(_lib.SmxError) as ei:
        _lib.check("smx_stack_fused_moe", _lib.SMX_ERR_WORKSPACE)
    assert ei.value.code == _lib.SMX_ERR_WORKSPACE
    assert "workspace" in str(ei.value)


def test_shared_workspace_size():
    ws, sws = L.smx_moe_workspace_size, L.smx_moe_shared_workspace_size
    assert sws(64, 2048, 1408, 60, 4, 0, 2) == ws(64, 2048, 1408, 60, 4, 2)
    assert sws(64, 2048, 1408, 60, 4, 5632, 2) > ws(64, 2048, 1408, 60, 4, 2)
    assert sws(128, 2048, 1408, 64, 6, 2816, 2) > sws(64, 2048, 1408, 64, 6, 2816, 2)
    assert sws(64, 2048, 1408, 60, 4, 100, 2) == 0    # shared I not a multiple of 128
    assert sws(64, 2048, 1408, 60, 4, -1, 2) == 0


def _shared(**kw):
    a = dict(hidden=A, out=A, dtype=2, T=4, H=256, logits=A, ldt=2, E=4, k=2, renorm=0, pool=A,
             slots=4, page=3 * 256 * 256, e2s=A, spage=A, sI=256, sgate=VP(0), scale=1.0,
             w=VP(0), ids=VP(0), ws=A, wsb=1 << 30, stream=VP(0))
    a.update(kw)
    return L.smx_fused_moe_shared_forward(
        a["hidden"], a["out"], a["dtype"], a["T"], a["H"], a["logits"], a["ldt"], a["E"], a["k"],
        a["renorm"], a["pool"], a["slots"], a["page"], a["e2s"], a["spage"], a["sI"], a["sgate"],
        a["scale"], a["w"], a["ids"], a["ws"], a["wsb"], a["stream"])


def test_shared_forward_rejects_before_launch():
    assert _shared(sI=-1) == _lib.SMX_ERR_INVALID_ARG
    assert _shared(spage=VP(0)) == _lib.SMX_ERR_INVALID_ARG              # I > 0 without a page
    assert _shared(sI=0) == _lib.SMX_ERR_INVALID_ARG                     # page without I
    assert _shared(sI=0, spage=VP(0), sgate=A) == _lib.SMX_ERR_INVALID_ARG  # gate, no expert
    assert _shared(scale=float("inf")) == _lib.SMX_ERR_INVALID_ARG
    assert _shared(scale=float("nan")) == _lib.SMX_ERR_INVALID_ARG
    assert _shared(spage=VP(0x10008)) == _lib.SMX_ERR_MISALIGNED
    assert _shared(sI=100) == _lib.SMX_ERR_UNSUPPORTED                   # not a multiple of 128
    assert _shared(wsb=16) == _lib.SMX_ERR_WORKSPACE
    assert _shared(T=0) == _lib.SMX_OK


def test_norm_gate_rejects_before_launch():
    f = L.smx_add_rmsnorm_gate
    #       hidden res out dt T  H    normw eps   gate E  logits stream
    base = [A, A, A, 2, 4, 256, A, 1e-6, A, 8, A, VP(0)]

    def call(**kw):
        a = list(base)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return f(*a)
    assert call(a3=7) == _lib.SMX_ERR_INVALID_ARG              # bad dtype
    assert call(a5=100) == _lib.SMX_ERR_UNSUPPORTED            # 200 bytes: not whole 16-byte vectors
    assert call(a5=32768) == _lib.SMX_ERR_UNSUPPORTED          # above the LDS-staged row limit
    assert call(a7=-1.0) == _lib.SMX_ERR_INVALID_ARG           # negative eps
    assert call(a7=float("nan")) == _lib.SMX_ERR_INVALID_ARG
    assert call(a9=0) == _lib.SMX_ERR_INVALID_ARG              # gate without experts
    assert call(a10=VP(0)) == _lib.SMX_ERR_INVALID_ARG         # gate without a logits buffer
    assert call(a9=300) == _lib.SMX_ERR_UNSUPPORTED
    assert call(a0=VP(0x10008)) == _lib.SMX_ERR_MISALIGNED
    assert call(a0=VP(0)) == _lib.SMX_ERR_INVALID_ARG
    assert call(a4=0) == _lib.SMX_OK
    # an empty batch's tensors may have null data pointers (torch's [0, n] tensors do)
    assert call(a4=0, a0=VP(0), a1=VP(0), a2=VP(0), a10=VP(0)) == _lib.SMX_OK


def test_layer_forward_rejects_before_launch():
    f = L.smx_moe_layer_forward
    #       hid res dt T H    nw eps  gw E k ren pool slots page e2s spage sI sgw scale lg w ids ws wsb stream
    base = [A, A, 2, 4, 256, A, 1e-6, A, 4, 2, 1, A, 4, 3 * 256 * 256, A, VP(0), 0, VP(0), 1.0,
            VP(0), VP(0), VP(0), A, 1 << 30, VP(0)]

    def call(**kw):
        a = list(base)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return f(*a)
    assert call(a9=5) == _lib.SMX_ERR_INVALID_ARG               # top_k > E
    assert call(a16=256) == _lib.SMX_ERR_INVALID_ARG            # shared I without a page
    assert call(a17=A) == _lib.SMX_ERR_INVALID_ARG              # shared gate without an expert
    assert call(a18=float("inf")) == _lib.SMX_ERR_INVALID_ARG
    assert call(a1=VP(0)) == _lib.SMX_ERR_INVALID_ARG           # the layer form needs a residual
    assert call(a7=VP(0)) == _lib.SMX_ERR_INVALID_ARG           # and a router gate
    assert call(a1=VP(0x10008)) == _lib.SMX_ERR_MISALIGNED
    assert call(a23=16) == _lib.SMX_ERR_WORKSPACE
    assert call(a3=0) == _lib.SMX_OK
    assert L.smx_moe_layer_workspace_size(32, 4096, 14336, 8, 2, 0, 2) > \
        L.smx_moe_workspace_size(32, 4096, 14336, 8, 2, 2)
    assert L.smx_moe_layer_workspace_size(32, 32768, 14336, 8, 2, 0, 2) == 0  # H above the norm limit


def test_transfer_entry_points_reject_bad_arguments():
    vp = VP()
    assert L.smx_host_alloc(0, ctypes.byref(vp)) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_host_free(None) == _lib.SMX_OK
    assert L.smx_h2d_engine_create(None) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_h2d_engine_destroy(None) == _lib.SMX_OK
    assert L.smx_h2d_submit(None, 4, b"t", A, A, 16, 2, 1, 0, VP(0)) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_h2d_wait(None, b"t", 0.0, None) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_h2d_has_task(None, b"t") == 0
    assert L.smx_h2d_clear(None, b"t") == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_h2d_set_enabled(None, 1) == _lib.SMX_ERR_INVALID_ARG
    assert L.smx_h2d_pending(None) == 0
    for code, word in [(1004, b"timed out"), (1005, b"no such")]:
        assert word in L.smx_error_string(code)


def test_transfer_engine_python_checks():
    import torch
    from ae_amd.backend import HtoDTransferEngine, TransferTaskType, TASK_PRIORITY_MAPPING
    eng = HtoDTransferEngine()
    assert not eng.has_task_id("x") and eng.wait_for_completion("x") is False
    with pytest.raises(RuntimeError):
        eng.submit_weight_loading_task(torch.zeros(4), torch.zeros(4), None, "t", 1, 0)
    assert [TASK_PRIORITY_MAPPING[t] for t in TransferTaskType] == [1, 2, 3, 4]
