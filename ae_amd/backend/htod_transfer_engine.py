"""Host -> device transfer engine with the reference's interface over the library's native
engine (one C++ worker thread, a priority queue of chunk copies, hipMemcpyAsync).

Reference: specmoe/backend/htod_transfer_engine.py:13-520. Task classes and their priority
order, chunked weight loading (one task per layer, ``num_chunks`` chunks, split by elements
with the remainder spread over the first chunks), ``wait_for_completion`` returning
``(success, execution_time)`` for weight tasks and ``success`` otherwise, ``clear_condition``,
and the worker's enable switch. Hidden-state and KV-cache loads are issued directly on the
caller's stream, as the reference does (its queued variants are unreachable there).
Streams must have the default priority.
"""
from __future__ import annotations

import ctypes
import logging
from enum import Enum
from typing import List, Optional, Tuple, Union

import torch

from .. import _lib

logger = logging.getLogger(__name__)


class TransferTaskType(Enum):
    HIDDEN_LOADING = _lib.SMX_H2D_HIDDEN
    KV_CACHE_LOADING = _lib.SMX_H2D_KV_CACHE
    DRAFT_KV_CACHE_LOADING = _lib.SMX_H2D_DRAFT_KV_CACHE
    WEIGHT_LOADING = _lib.SMX_H2D_WEIGHT


# smaller number = more urgent (the native queue orders by this, then layer, then chunk)
TASK_PRIORITY_MAPPING = {
    TransferTaskType.HIDDEN_LOADING: 1,
    TransferTaskType.KV_CACHE_LOADING: 2,
    TransferTaskType.DRAFT_KV_CACHE_LOADING: 3,
    TransferTaskType.WEIGHT_LOADING: 4,
}


def _check_pair(src: torch.Tensor, dst: torch.Tensor) -> None:
    if src.device.type != "cpu" or dst.device.type != "cuda":
        raise ValueError("expected a host source tensor and a GPU destination tensor")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("source and destination must be contiguous")
    if src.numel() * src.element_size() != dst.numel() * dst.element_size():
        raise ValueError("source and destination sizes differ")


class HtoDTransferEngine:
    """Host-to-device transfer engine (see module docstring)."""

    def __init__(self, chunk_size: int = 1024 * 1024):
        self.chunk_size = chunk_size
        self.running = False
        self._engine = None
        self._tasks = {}  # task id -> kind, to shape wait_for_completion's result
        self._keep = {}   # task id -> (src, dst): tensors stay alive while chunks are queued

    # -- lifecycle -------------------------------------------------------------------------
    def start(self):
        if self.running:
            logger.warning("HtoDTransferEngine is already running")
            return
        h = ctypes.c_void_p()
        _lib.check("smx_h2d_engine_create", _lib.lib().smx_h2d_engine_create(ctypes.byref(h)))
        self._engine = h
        self.running = True

    def stop(self):
        if not self.running:
            return
        self.running = False
        _lib.lib().smx_h2d_engine_destroy(self._engine)
        self._engine = None
        self._tasks.clear()
        self._keep.clear()

    def __del__(self):
        try:
            self.stop()
        except Exception:
            pass

    # -- submission ------------------------------------------------------------------------
    def submit_hidden_loading_task(self, src: torch.Tensor, dst: torch.Tensor,
                                   stream: torch.cuda.Stream, event: torch.cuda.Event):
        """Direct copy on `stream`, then `event` recorded (reference :233-240)."""
        with torch.cuda.stream(stream):
            dst.copy_(src, non_blocking=True)
            event.record(stream)

    def submit_weight_loading_task(self, src: torch.Tensor, dst: torch.Tensor,
                                   stream: torch.cuda.Stream, task_id: str, num_chunks: int,
                                   layer_id: int):
        self._submit_chunked_task(TransferTaskType.WEIGHT_LOADING, src, dst, stream, task_id,
                                  num_chunks, layer_id)

    def submit_draft_kv_cache_loading_task(self, src: torch.Tensor, dst: torch.Tensor,
                                           stream: torch.cuda.Stream, task_id: str,
                                           num_chunks: int, layer_id: int = 0):
        self._submit_chunked_task(TransferTaskType.DRAFT_KV_CACHE_LOADING, src, dst, stream,
                                  task_id, num_chunks, layer_id)

    def _submit_chunked_task(self, task_type: TransferTaskType, src: torch.Tensor,
                             dst: torch.Tensor, stream: torch.cuda.Stream, task_id: str,
                             num_chunks: int, layer_id: int):
        if not self.running:
            raise RuntimeError("HtoDTransferEngine is not running")
        _check_pair(src, dst)
        rc = _lib.lib().smx_h2d_submit(
            self._engine, task_type.value, task_id.encode(), ctypes.c_void_p(dst.data_ptr()),
            ctypes.c_void_p(src.data_ptr()), src.numel() * src.element_size(), src.element_size(),
            int(num_chunks), int(layer_id), ctypes.c_void_p(stream.cuda_stream))
        _lib.check("smx_h2d_submit", rc)
        self._tasks[task_id] = task_type
        self._keep[task_id] = (src, dst)

    # -- completion ------------------------------------------------------------------------
    def has_task_id(self, task_id: str) -> bool:
        return bool(self.running and _lib.lib().smx_h2d_has_task(self._engine, task_id.encode()))

    def wait_for_completion(self, task_id: str, timeout: Optional[float] = None
                            ) -> Union[bool, Tuple[bool, Optional[float]]]:
        """Weight tasks: (True, seconds from the first chunk's start to the last chunk's end)
        once the last chunk has landed, (False, None) if a copy failed; other tasks: True /
        False. An unknown id or a timeout returns False (reference :375-411)."""
        if not self.running:
            return False
        secs = ctypes.c_double(-1.0)
        rc = _lib.lib().smx_h2d_wait(self._engine, task_id.encode(),
                                     -1.0 if timeout is None else float(timeout), ctypes.byref(secs))
        if rc == _lib.SMX_ERR_NOT_FOUND:
            logger.warning(f"task id {task_id} does not exist")
            return False
        if rc == _lib.SMX_ERR_TIMEOUT:
            logger.warning(f"task {task_id} timed out")
            return False
        ok = rc == _lib.SMX_OK
        if self._tasks.get(task_id) == TransferTaskType.WEIGHT_LOADING:
            return ok, (secs.value if ok else None)
        return ok

    def clear_condition(self, task_ids: List[str]):
        for task_id in task_ids:
            if self.running:
                _lib.lib().smx_h2d_clear(self._engine, task_id.encode())
            self._tasks.pop(task_id, None)
            self._keep.pop(task_id, None)

    # -- worker switch (the reference's worker_enabled) ---------------------------------------
    def set_worker_enabled(self, enabled: bool):
        _lib.check("smx_h2d_set_enabled", _lib.lib().smx_h2d_set_enabled(self._engine, int(enabled)))

    def pending_chunks(self) -> int:
        return int(_lib.lib().smx_h2d_pending(self._engine)) if self.running else 0
