"""Fused MoE operators on MI355X: the functions of specmoe/layers/fused_moe_kernel.py.

``moe_align_block_size`` and ``stack_fused_moe`` keep the reference's names, arguments,
return values and assertions; the work runs in libspecmoe_mi355x.so (HIP, gfx950).
``fused_moe_forward`` is routing + experts in one library call, used by FusedMoE.forward.

Expert pool contract (specmoe/layers/FusedMoE.py:485-505 packs it; the pool is allocated at
specmoe/backend/execution_engine.py:1189): ``w1`` is ``[P, 3*I*H]``, each page holding
``[W1 gate (I x H) | W3 up (I x H) | W2 down (H x I)]`` row-major, and ``indicies[e]`` (int64,
on the GPU) names the page of expert ``e``. Only the pages of routed experts are read.
"""
from __future__ import annotations

import contextlib
from typing import Iterator, Optional, Tuple

import torch

from .. import _lib
from ._torch import dtype_code, ptr, require_gpu, stream_of, workspace


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int,
                         num_experts: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sort flat assignments by expert and pad each expert's run to a multiple of block_size.

    Reference: specmoe/layers/fused_moe_kernel.py:16-85. Returns
    ``(sorted_token_ids, expert_ids, num_tokens_post_padded)`` with the reference's sizes:
    ``sorted_token_ids`` has ``numel + E*(block_size-1)`` entries, padding holds ``numel``;
    ``expert_ids`` has ``cdiv(len(sorted_token_ids), block_size)`` entries, the expert of each
    block (entries past ``num_tokens_post_padded / block_size`` are -1 here; the reference
    leaves them unset). Within an expert, flat indices appear in ascending order.
    """
    require_gpu(topk_ids)
    ids = topk_ids.contiguous()
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    numel = ids.numel()
    max_num_tokens_padded = numel + num_experts * (block_size - 1)
    sorted_ids = torch.empty((max_num_tokens_padded,), dtype=torch.int32, device=ids.device)
    max_num_m_blocks = (max_num_tokens_padded + block_size - 1) // block_size
    expert_ids = torch.empty((max_num_m_blocks,), dtype=torch.int32, device=ids.device)
    num_tokens_post_pad = torch.empty((1,), dtype=torch.int32, device=ids.device)
    _lib.call("smx_moe_align_block_size", ptr(ids), numel, num_experts, block_size,
              ptr(sorted_ids), ptr(expert_ids), ptr(num_tokens_post_pad), stream_of(ids))
    return sorted_ids, expert_ids, num_tokens_post_pad


def set_tiled_min_tokens(tokens_per_expert: Optional[int]) -> int:
    """Set the expected tokens per active expert at which MoE calls switch from the
    weight-streaming expert kernels to the tiled MFMA kernels (0: always tiled; None: the
    library default). Returns the previous setting. Process-wide."""
    prev = int(_lib.lib().smx_tiled_min_tokens())
    _lib.call("smx_set_tiled_min_tokens", -1 if tokens_per_expert is None else int(tokens_per_expert))
    return prev


@contextlib.contextmanager
def tiled_min_tokens(tokens_per_expert: Optional[int]) -> Iterator[None]:
    """Scope a set_tiled_min_tokens setting (restored on exit)."""
    prev = set_tiled_min_tokens(tokens_per_expert)
    try:
        yield
    finally:
        set_tiled_min_tokens(prev)


def set_fused_down_max_tokens(tokens: Optional[int]) -> int:
    """Set the largest batch (tokens) whose down projection and top-k combine run as one
    kernel (0: never; at most 8; None: the library's default rule, which fuses batches whose
    output rows each stream at most 48 KB of weight rows). Returns the previous setting (None
    for the default rule). Process-wide."""
    prev = int(_lib.lib().smx_fused_down_max_tokens())
    _lib.call("smx_set_fused_down_max_tokens", -1 if tokens is None else int(tokens))
    return None if prev < 0 else prev


@contextlib.contextmanager
def fused_down_max_tokens(tokens: Optional[int]) -> Iterator[None]:
    """Scope a set_fused_down_max_tokens setting (restored on exit)."""
    prev = set_fused_down_max_tokens(tokens)
    try:
        yield
    finally:
        set_fused_down_max_tokens(prev)


def set_fp32_gemm_outputs_fp16(on: bool) -> bool:
    """fp32 runs: round the routed GEMM outputs (gate/up and the weighted down projection) to
    fp16 as the reference stores them for fp32 inputs (specmoe/layers/fused_moe_kernel.py:
    203,248), instead of keeping true fp32. Returns the previous setting. Process-wide."""
    prev = bool(_lib.lib().smx_fp32_gemm_outputs_fp16())
    _lib.call("smx_set_fp32_gemm_outputs_fp16", 1 if on else 0)
    return prev


@contextlib.contextmanager
def fp32_gemm_outputs_fp16(on: bool = True) -> Iterator[None]:
    """Scope a set_fp32_gemm_outputs_fp16 setting (restored on exit)."""
    prev = set_fp32_gemm_outputs_fp16(on)
    try:
        yield
    finally:
        set_fp32_gemm_outputs_fp16(prev)


def set_routing_in_gateup(on: bool) -> bool:
    """Route small batches inside the gate/up launch (default) or with the routing kernels.
    Returns the previous setting. Process-wide."""
    prev = bool(_lib.lib().smx_routing_in_gateup())
    _lib.call("smx_set_routing_in_gateup", 1 if on else 0)
    return prev


@contextlib.contextmanager
def routing_in_gateup(on: bool) -> Iterator[None]:
    """Scope a set_routing_in_gateup setting (restored on exit)."""
    prev = set_routing_in_gateup(on)
    try:
        yield
    finally:
        set_routing_in_gateup(prev)


def set_gateup_waves(waves: Optional[int]) -> Optional[int]:
    """Set the waves per workgroup of the weight-streaming gate/up kernel (4, 2 or 1; None: the
    library's rule, which uses 2 -- twice the workgroups -- when a 4-wave grid would put two
    workgroups on some CUs and one on most, and for many-expert blocks of hidden rows up to 4 KB
    with grids of 1.25+ residencies splits each item's K walk between wave pairs). Outputs do
    not depend on the forced settings 4, 2 and 1; the rule's K split sums in another fixed order.
    Returns the previous setting (None for the rule). Process-wide."""
    prev = int(_lib.lib().smx_gateup_waves())
    _lib.call("smx_set_gateup_waves", 0 if waves is None else int(waves))
    return None if prev == 0 else prev


@contextlib.contextmanager
def gateup_waves(waves: Optional[int]) -> Iterator[None]:
    """Scope a set_gateup_waves setting (restored on exit)."""
    prev = set_gateup_waves(waves)
    try:
        yield
    finally:
        set_gateup_waves(prev)


def set_gateup_item_walk(on: bool) -> bool:
    """Let gate/up grids larger than one residency of the chip run as workgroups that walk
    several work items (default) or launch one workgroup per item. Outputs do not depend on
    it. Returns the previous setting. Process-wide."""
    prev = bool(_lib.lib().smx_gateup_item_walk())
    _lib.call("smx_set_gateup_item_walk", 1 if on else 0)
    return prev


@contextlib.contextmanager
def gateup_item_walk(on: bool) -> Iterator[None]:
    """Scope a set_gateup_item_walk setting (restored on exit)."""
    prev = set_gateup_item_walk(on)
    try:
        yield
    finally:
        set_gateup_item_walk(prev)


def _caller_buffers(hidden_states: torch.Tensor, inplace: bool, out: Optional[torch.Tensor],
                    ws: Optional[torch.Tensor], nbytes: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The output and workspace of a call: the caller's when given (checked), else the input
    itself (inplace) or a new tensor, and a workspace from the caching allocator."""
    if out is None:
        out = hidden_states if inplace else torch.empty_like(hidden_states)
    else:
        assert not inplace, "out= and inplace=True both name the output"
        assert out.shape == hidden_states.shape and out.dtype == hidden_states.dtype, \
            "out must match hidden_states in shape and dtype"
        assert out.is_contiguous() and out.device == hidden_states.device, \
            "out must be contiguous and on the device of hidden_states"
    if ws is None:
        ws = workspace(nbytes, hidden_states.device)
    else:
        assert ws.dtype == torch.uint8 and ws.is_contiguous() and ws.device == hidden_states.device, \
            "workspace must be a contiguous uint8 tensor on the device of hidden_states"
        assert ws.numel() >= nbytes, f"workspace holds {ws.numel()} bytes, the call needs {nbytes}"
    return out, ws


def _pool_geometry(hidden_states: torch.Tensor, w1: torch.Tensor) -> Tuple[int, int]:
    H = hidden_states.shape[1]
    _, page_size = w1.shape
    assert page_size % (3 * H) == 0, "pool page is not 3*I*H elements"
    return H, page_size // (3 * H)


def _as_index(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    t = t.contiguous()
    return t if t.dtype == dtype else t.to(dtype)


def stack_fused_moe(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    indicies: torch.Tensor,
    gating_output: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    renormalize: bool,
    inplace: bool = False,
) -> torch.Tensor:
    """MoE experts over a pooled weight cache, routing given.

    Reference: specmoe/layers/fused_moe_kernel.py:253-349. ``y[t] = sum_j w[t,j] *
    W2_e(silu(W1_e x_t) * W3_e x_t)`` with e = topk_ids[t,j] and expert e's weights in page
    ``indicies[e]`` of ``w1``. With ``inplace`` the result is written into hidden_states
    (the reference's ``torch.sum(..., out=hidden_states)``) and hidden_states is returned.
    ``renormalize`` is accepted for signature parity; like the reference, the weights are
    used as given.
    """
    # Check constraints (same as the reference).
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    E = gating_output.shape[1]
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert hidden_states.dtype in [torch.float32, torch.float16, torch.bfloat16]
    assert w1.dtype == hidden_states.dtype, "expert pool and hidden states dtypes differ"
    require_gpu(hidden_states, w1, indicies, topk_weights, topk_ids)
    H, I = _pool_geometry(hidden_states, w1)
    T = hidden_states.shape[0]
    top_k = topk_ids.shape[1]
    out = hidden_states if inplace else torch.empty_like(hidden_states)
    slots = _as_index(indicies, torch.int64)
    ids = _as_index(topk_ids, torch.int32)
    w = _as_index(topk_weights, torch.float32)
    dt = dtype_code(hidden_states.dtype)
    nbytes = _lib.lib().smx_moe_workspace_size(T, H, I, E, top_k, dt)
    if nbytes == 0 and T > 0:
        raise ValueError(f"unsupported MoE shape T={T} H={H} I={I} E={E} top_k={top_k}")
    ws = workspace(nbytes, hidden_states.device)
    _lib.call("smx_stack_fused_moe", ptr(hidden_states), ptr(out), dt, T, H, ptr(w1),
              w1.shape[0], w1.shape[1], ptr(slots), E, ptr(w), ptr(ids), top_k,
              ptr(ws), ws.numel(), stream_of(hidden_states))
    return out


def fused_moe_forward(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    w1: torch.Tensor,
    indicies: torch.Tensor,
    top_k: int,
    renormalize: bool,
    inplace: bool = True,
    return_routing: bool = False,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
):
    """Routing (select_experts) and stack_fused_moe in one library call.

    Reference: the body of UnquantizedFusedMoEMethod.forward_cuda,
    specmoe/layers/FusedMoE.py:155-196 (select_experts at :174, stack_fused_moe at :187,
    inplace=True). With ``return_routing`` also returns ``(topk_weights, topk_ids)``.
    ``out`` (with ``inplace=False``) receives the result; ``workspace`` is a caller-owned uint8
    scratch of at least ``smx_moe_workspace_size`` bytes (default: one from torch's caching
    allocator). Neither needs any initial contents: the call writes every byte it reads.
    """
    assert hidden_states.shape[0] == router_logits.shape[0], "Number of tokens mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert hidden_states.dtype in [torch.float32, torch.float16, torch.bfloat16]
    assert w1.dtype == hidden_states.dtype, "expert pool and hidden states dtypes differ"
    require_gpu(hidden_states, router_logits, w1, indicies)
    H, I = _pool_geometry(hidden_states, w1)
    T, E = router_logits.shape
    logits = router_logits.contiguous()
    slots = _as_index(indicies, torch.int64)
    dt = dtype_code(hidden_states.dtype)
    nbytes = _lib.lib().smx_moe_workspace_size(T, H, I, E, top_k, dt)
    if nbytes == 0 and T > 0:
        raise ValueError(f"unsupported MoE shape T={T} H={H} I={I} E={E} top_k={top_k}")
    out, ws = _caller_buffers(hidden_states, inplace, out, workspace, nbytes)
    w = ids = None
    if return_routing:
        w = torch.empty((T, top_k), dtype=torch.float32, device=hidden_states.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=hidden_states.device)
    _lib.call("smx_fused_moe_forward", ptr(hidden_states), ptr(out), dt, T, H, ptr(logits),
              dtype_code(logits.dtype), E, top_k, int(bool(renormalize)), ptr(w1), w1.shape[0],
              w1.shape[1], ptr(slots), ptr(w), ptr(ids), ptr(ws), ws.numel(),
              stream_of(hidden_states))
    if return_routing:
        return out, w, ids
    return out


def _shared_terms(hidden_states: torch.Tensor, shared_w: Optional[torch.Tensor],
                  shared_gate_logits: Optional[torch.Tensor], T: int, H: int,
                  gate_dtype: torch.dtype):
    """-> (shared_I, contiguous gate logits or None), checking the shared expert's operands."""
    Is = 0
    if shared_w is not None:
        assert shared_w.is_contiguous(), "shared expert weights must be contiguous"
        assert shared_w.dtype == hidden_states.dtype, "shared expert and hidden states dtypes differ"
        assert shared_w.numel() % (3 * H) == 0, "shared expert page is not 3*Is*H elements"
        Is = shared_w.numel() // (3 * H)
    sgate = None
    if shared_gate_logits is not None:
        assert shared_w is not None, "a shared-expert gate needs a shared expert"
        assert shared_gate_logits.numel() == T, "one shared-expert gate logit per token"
        assert shared_gate_logits.dtype == gate_dtype, \
            f"shared-expert gate logits must be {gate_dtype}"
        sgate = shared_gate_logits.contiguous()
    return Is, sgate


def fused_moe_shared_forward(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    w1: torch.Tensor,
    indicies: torch.Tensor,
    top_k: int,
    renormalize: bool,
    shared_w: Optional[torch.Tensor],
    shared_gate_logits: Optional[torch.Tensor] = None,
    routed_scaling_factor: float = 1.0,
    inplace: bool = True,
    return_routing: bool = False,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
):
    """A MoE block with an always-active shared expert, in one library call.

    ``y = round(round(routed * routed_scaling_factor) + s * shared)`` where ``routed`` is
    :func:`fused_moe_forward`'s result, ``shared`` the SwiGLU MLP whose weights are packed in
    ``shared_w`` like one pool page (``[W1s | W3s | W2s]``, ``3*Is*H`` elements) and ``s`` is
    ``sigmoid(shared_gate_logits)`` (``[T]`` or ``[T,1]``) or 1. The reference has no shared
    expert; this is the block of Qwen1.5-MoE (gated shared expert) and DeepSeek-V2 (ungated,
    ``n_shared * I`` columns, scaled routed output) over the routed path of
    specmoe/layers/FusedMoE.py:155-196. ``out`` and ``workspace`` as in
    :func:`fused_moe_forward` (the workspace size is ``smx_moe_shared_workspace_size``).
    """
    assert hidden_states.shape[0] == router_logits.shape[0], "Number of tokens mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert hidden_states.dtype in [torch.float32, torch.float16, torch.bfloat16]
    assert w1.dtype == hidden_states.dtype, "expert pool and hidden states dtypes differ"
    require_gpu(hidden_states, router_logits, w1, indicies, shared_w, shared_gate_logits)
    H, I = _pool_geometry(hidden_states, w1)
    T, E = router_logits.shape
    Is, sgate = _shared_terms(hidden_states, shared_w, shared_gate_logits, T, H, router_logits.dtype)
    logits = router_logits.contiguous()
    slots = _as_index(indicies, torch.int64)
    dt = dtype_code(hidden_states.dtype)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, E, top_k, Is, dt)
    if nbytes == 0 and T > 0:
        raise ValueError(f"unsupported MoE shape T={T} H={H} I={I} E={E} top_k={top_k} "
                         f"shared I={Is}")
    out, ws = _caller_buffers(hidden_states, inplace, out, workspace, nbytes)
    w = ids = None
    if return_routing:
        w = torch.empty((T, top_k), dtype=torch.float32, device=hidden_states.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=hidden_states.device)
    _lib.call("smx_fused_moe_shared_forward", ptr(hidden_states), ptr(out), dt, T, H, ptr(logits),
              dtype_code(logits.dtype), E, top_k, int(bool(renormalize)), ptr(w1), w1.shape[0],
              w1.shape[1], ptr(slots), ptr(shared_w), Is, ptr(sgate), float(routed_scaling_factor),
              ptr(w), ptr(ids), ptr(ws), ws.numel(), stream_of(hidden_states))
    if return_routing:
        return out, w, ids
    return out


def stack_fused_moe_shared(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    indicies: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    shared_w: Optional[torch.Tensor],
    shared_gate_logits: Optional[torch.Tensor] = None,
    routed_scaling_factor: float = 1.0,
    inplace: bool = True,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """:func:`fused_moe_shared_forward` on the caller's routing (``topk_weights`` /
    ``topk_ids`` as :func:`stack_fused_moe` takes them), for blocks whose routing is not the
    plain top-k softmax (DeepSeek-V2's group-limited and DeepSeek-V3's biased top-k,
    :func:`ae_amd.layers.grouped_topk`). ``shared_gate_logits`` are in the activations' dtype.
    One library call (``smx_stack_fused_moe_shared``)."""
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert hidden_states.dtype in [torch.float32, torch.float16, torch.bfloat16]
    assert w1.dtype == hidden_states.dtype, "expert pool and hidden states dtypes differ"
    assert topk_weights.shape == topk_ids.shape, "topk shape mismatch"
    assert topk_ids.shape[0] == hidden_states.shape[0], "Number of tokens mismatch"
    require_gpu(hidden_states, w1, indicies, topk_weights, topk_ids, shared_w, shared_gate_logits)
    H, I = _pool_geometry(hidden_states, w1)
    T, top_k = topk_ids.shape
    E = indicies.numel()
    Is, sgate = _shared_terms(hidden_states, shared_w, shared_gate_logits, T, H, hidden_states.dtype)
    slots = _as_index(indicies, torch.int64)
    ids = _as_index(topk_ids, torch.int32)
    w = _as_index(topk_weights, torch.float32)
    dt = dtype_code(hidden_states.dtype)
    nbytes = _lib.lib().smx_moe_shared_workspace_size(T, H, I, E, top_k, Is, dt)
    if nbytes == 0 and T > 0:
        raise ValueError(f"unsupported MoE shape T={T} H={H} I={I} E={E} top_k={top_k} "
                         f"shared I={Is}")
    out, ws = _caller_buffers(hidden_states, inplace, out, workspace, nbytes)
    _lib.call("smx_stack_fused_moe_shared", ptr(hidden_states), ptr(out), dt, T, H, ptr(w1),
              w1.shape[0], w1.shape[1], ptr(slots), E, ptr(w), ptr(ids), top_k, ptr(shared_w), Is,
              ptr(sgate), float(routed_scaling_factor), ptr(ws), ws.numel(),
              stream_of(hidden_states))
    return out
