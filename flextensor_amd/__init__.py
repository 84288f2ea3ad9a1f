"""MI355X-native weight streaming behind FlexTensor's offload API.

Host logic (planning, scheduling, the offload phases) is Python over PyTorch;
device work goes through the HIP C-ABI library ``libftx_hip.so``
(``include/ftx.h``): pinned host arenas, host-to-device copy engines
(hipMemcpyAsync and a zero-copy kernel), a batched scatter kernel and
hipEvent gating.
"""

__version__ = "0.1.0"

from .config import OffloadConfig, load_config_from_env  # noqa: E402
from .manager import (  # noqa: E402
    DEFAULT_MANAGER_NAME,
    GPUMemoryUsage,
    OffloadManager,
    OffloadPhase,
    collect_offload_timing,
    get_gpu_memory_usage,
    get_offload_manager,
    load_profile,
    offload,
    offload_from_profile,
    offload_from_state,
    release,
    reset_offload_timing,
    save_profile,
)
from .profile import TensorManagerState, load_state, save_state  # noqa: E402
from .shared_offload import SharedOffloadSession  # noqa: E402

__all__ = [
    "DEFAULT_MANAGER_NAME",
    "GPUMemoryUsage",
    "OffloadConfig",
    "OffloadManager",
    "OffloadPhase",
    "SharedOffloadSession",
    "TensorManagerState",
    "collect_offload_timing",
    "get_gpu_memory_usage",
    "get_offload_manager",
    "load_config_from_env",
    "load_profile",
    "load_state",
    "offload",
    "offload_from_profile",
    "offload_from_state",
    "release",
    "reset_offload_timing",
    "save_profile",
    "save_state",
]
