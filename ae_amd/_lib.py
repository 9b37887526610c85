"""ctypes binding of libspecmoe_mi355x.so (the C ABI in include/specmoe_mi355x.h).

The library is built in-tree by ``ae_amd.build``. Loading fails loudly when it is missing:
there is no fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

SMX_F32, SMX_F16, SMX_BF16 = 0, 1, 2
SMX_OK = 0
SMX_ERR_INVALID_ARG = 1000
SMX_ERR_UNSUPPORTED = 1001
SMX_ERR_WORKSPACE = 1002
SMX_ERR_MISALIGNED = 1003
SMX_ERR_TIMEOUT = 1004
SMX_ERR_NOT_FOUND = 1005
SMX_ERR_SCRATCH = 1006
SMX_NOALLOC_SCRATCH_BYTES = 32 << 20
SMX_H2D_HIDDEN, SMX_H2D_KV_CACHE, SMX_H2D_DRAFT_KV_CACHE, SMX_H2D_WEIGHT = 1, 2, 3, 4

# (name, restype, argtypes) of every exported entry point, in header order.
_c_void_p, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
SIGNATURES = [
    ("smx_version", ctypes.c_int, []),
    ("smx_error_string", ctypes.c_char_p, [_i32]),
    ("smx_topk_softmax", ctypes.c_int,
     [_c_void_p, _i32, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p]),
    ("smx_grouped_topk", ctypes.c_int,
     [_c_void_p, _i32, _i64, _i64, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
      _c_void_p]),
    ("smx_moe_align_block_size", ctypes.c_int,
     [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    ("smx_moe_workspace_size", _sz, [_i64, _i64, _i64, _i64, _i64, _i32]),
    ("smx_stack_fused_moe", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
      _c_void_p, _c_void_p, _i64, _c_void_p, _sz, _c_void_p]),
    ("smx_stack_fused_moe_shared", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
      _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_float, _c_void_p, _sz,
      _c_void_p]),
    ("smx_fused_moe_forward", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _i32, _i64, _i64, _i32,
      _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p]),
    ("smx_fused_moe_forward_noalloc", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _i32, _i64, _i64, _i32,
      _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    ("smx_moe_shared_workspace_size", _sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    ("smx_fused_moe_shared_forward", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _i32, _i64, _i64, _i32,
      _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, ctypes.c_float,
      _c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p]),
    ("smx_add_rmsnorm_gate", ctypes.c_int,
     [_c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, ctypes.c_float, _c_void_p,
      _i64, _c_void_p, _c_void_p]),
    ("smx_moe_layer_workspace_size", _sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    ("smx_moe_layer_forward", ctypes.c_int,
     [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, ctypes.c_float, _c_void_p, _i64, _i64,
      _i32, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, ctypes.c_float,
      _c_void_p, _c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p]),
    ("smx_host_alloc", ctypes.c_int, [_sz, ctypes.POINTER(_c_void_p)]),
    ("smx_host_free", ctypes.c_int, [_c_void_p]),
    ("smx_h2d_engine_create", ctypes.c_int, [ctypes.POINTER(_c_void_p)]),
    ("smx_h2d_engine_destroy", ctypes.c_int, [_c_void_p]),
    ("smx_h2d_submit", ctypes.c_int,
     [_c_void_p, _i32, ctypes.c_char_p, _c_void_p, _c_void_p, _sz, _sz, _i64, _i64, _c_void_p]),
    ("smx_h2d_wait", ctypes.c_int,
     [_c_void_p, ctypes.c_char_p, ctypes.c_double, ctypes.POINTER(ctypes.c_double)]),
    ("smx_h2d_has_task", ctypes.c_int, [_c_void_p, ctypes.c_char_p]),
    ("smx_h2d_clear", ctypes.c_int, [_c_void_p, ctypes.c_char_p]),
    ("smx_h2d_set_enabled", ctypes.c_int, [_c_void_p, _i32]),
    ("smx_h2d_pending", ctypes.c_int, [_c_void_p]),
    ("smx_set_tiled_min_tokens", ctypes.c_int, [_i64]),
    ("smx_tiled_min_tokens", _i64, []),
    ("smx_set_fused_down_max_tokens", ctypes.c_int, [_i64]),
    ("smx_fused_down_max_tokens", _i64, []),
    ("smx_set_fp32_gemm_outputs_fp16", ctypes.c_int, [_i32]),
    ("smx_fp32_gemm_outputs_fp16", _i32, []),
    ("smx_set_routing_in_gateup", ctypes.c_int, [_i32]),
    ("smx_routing_in_gateup", _i32, []),
    ("smx_set_gateup_waves", ctypes.c_int, [_i32]),
    ("smx_gateup_waves", _i32, []),
    ("smx_set_gateup_item_walk", ctypes.c_int, [_i32]),
    ("smx_gateup_item_walk", _i32, []),
    ("smx_set_gateup_expert_items", ctypes.c_int, [_i32]),
    ("smx_gateup_expert_items", _i32, []),
    ("smx_set_single_launch_layer", ctypes.c_int, [_i32]),
    ("smx_single_launch_layer", _i32, []),
    ("smx_set_layer_sync_test", ctypes.c_int, [_i32, _i64]),
    ("smx_moe_plan_info", ctypes.c_int,
     [_i64, _i64, _i64, _i64, _i64, _i64, _i32, ctypes.POINTER(_i64), _i32]),
    ("smx_set_profile_events", ctypes.c_int, [ctypes.POINTER(_c_void_p), _i32]),
    ("smx_stream_read", ctypes.c_int, [_c_void_p, _sz, _sz, _c_void_p, _c_void_p]),
]

_lock = threading.Lock()
_lib = None


class SmxError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m ae_amd.build` "
                    "(the MoE path has no fallback implementation)")
            # PyTorch-ROCm wheels ship their own HIP runtime (libamdhip64.so, SONAME
            # libamdhip64.so.7). Importing torch first maps it, so this library's
            # DT_NEEDED libamdhip64.so.7 binds to that same runtime. Loaded the other way
            # round, torch would map a second runtime and kernels launched here could not
            # see torch's device context.
            import torch  # noqa: F401
            handle = ctypes.CDLL(LIB_PATH)
            for name, restype, argtypes in SIGNATURES:
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


# Fields of smx_moe_plan_info, in the order of enum smx_plan_field.
PLAN_FIELDS = ("tiled", "fused_down", "span", "max_ranges", "tok_tiles", "splits", "split_steps",
               "down_rows", "gateup_waves", "gateup_ksplit", "shared_splits",
               "shared_split_steps", "shared_tok_groups", "shared_gateup_blocks",
               "shared_down_blocks", "tile_gateup_grid", "tile_down_grid", "single_launch",
               "sync_blocks", "sync_offset", "topk_in_gateup", "expert_items", "chunk_tokens",
               "workspace_bytes")


def plan_info(T: int, H: int, I: int, E: int, top_k: int, dtype: int, shared_I: int = 0) -> dict:
    """The launch plan of a MoE call of these sizes under the current settings (host only)."""
    out = (ctypes.c_int64 * len(PLAN_FIELDS))()
    n = lib().smx_moe_plan_info(T, H, I, E, top_k, shared_I, dtype, out, len(PLAN_FIELDS))
    if n >= 1000:
        check("smx_moe_plan_info", n)
    assert n == len(PLAN_FIELDS), f"library reports {n} plan fields, binding knows {len(PLAN_FIELDS)}"
    return dict(zip(PLAN_FIELDS, (int(v) for v in out)))


def check(fn: str, code: int) -> None:
    if code != SMX_OK:
        msg = lib().smx_error_string(code).decode()
        raise SmxError(fn, code, msg)


def call(fn: str, *args) -> None:
    """Invoke entry point `fn` and raise SmxError on a non-zero status."""
    check(fn, getattr(lib(), fn)(*args))
