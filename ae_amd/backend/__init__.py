"""Host-side services around the MoE path: pinned host memory and host -> device streaming
of expert pages (the reference's specmoe/backend pin_memory_allocator and
htod_transfer_engine), on the library's HIP runtime."""
from .htod_transfer_engine import TASK_PRIORITY_MAPPING, HtoDTransferEngine, TransferTaskType
from .pin_memory_allocator import (cuda_host_alloc, free_pinned_tensor, make_pinned_numpy_array,
                                   make_pinned_tensor)

__all__ = ["HtoDTransferEngine", "TransferTaskType", "TASK_PRIORITY_MAPPING", "cuda_host_alloc",
           "make_pinned_numpy_array", "make_pinned_tensor", "free_pinned_tensor"]
