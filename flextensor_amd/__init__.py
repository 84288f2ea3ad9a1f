"""MI355X-native weight streaming behind FlexTensor's offload API.

Host logic (planning, scheduling, the offload phases) is Python over PyTorch;
device work goes through the HIP C-ABI library ``libftx_hip.so``
(``include/ftx.h``): pinned host arenas, host-to-device copy engines
(hipMemcpyAsync and a zero-copy kernel), a batched scatter kernel and
hipEvent gating, an fp8-weight MFMA GEMM, and a staged copy engine for
pageable and shared-memory sources. Models can be built straight from a
saved profile and a safetensors checkpoint (``load_model_from_profile``).
"""

__version__ = "0.1.0"

from .config import (  # noqa: E402
    OffloadConfig,
    PinnedMemoryMode,
    load_config,
    load_config_from_env,
    load_config_from_file,
)
from .lazy_model_init import load_model_from_profile  # noqa: E402
from .manager import (  # noqa: E402
    DEFAULT_MANAGER_NAME,
    GPUMemoryUsage,
    OffloadBlock,
    OffloadManager,
    OffloadPhase,
    clear_profiling_durations,
    collect_offload_timing,
    get_gpu_memory_usage,
    get_offload_manager,
    init,
    load_profile,
    offload,
    offload_block,
    offload_from_profile,
    offload_from_state,
    offload_units,
    pause_profiling,
    release,
    request_strategy_replan,
    reset_offload_timing,
    resident_units,
    resume_profiling,
    save_profile,
    set_config,
    suspend_profiling,
    update_offload_timing,
    update_state,
)
from .profile import TensorManagerState, load_state, save_state  # noqa: E402
from .replan import StrategyReplanStatus  # noqa: E402
from .shared_offload import (  # noqa: E402
    SharedOffloadSession,
    ShmCoordinatorError,
    ShmCreatorDiedError,
    ShmCreatorFailedError,
)
from .timing import OffloadTimingReport, OffloadTimingSnapshot, format_offload_timing_table  # noqa: E402

__all__ = [
    "DEFAULT_MANAGER_NAME",
    "GPUMemoryUsage",
    "OffloadBlock",
    "OffloadConfig",
    "OffloadManager",
    "OffloadPhase",
    "OffloadTimingReport",
    "OffloadTimingSnapshot",
    "PinnedMemoryMode",
    "SharedOffloadSession",
    "ShmCoordinatorError",
    "ShmCreatorDiedError",
    "ShmCreatorFailedError",
    "StrategyReplanStatus",
    "TensorManagerState",
    "clear_profiling_durations",
    "collect_offload_timing",
    "format_offload_timing_table",
    "get_gpu_memory_usage",
    "get_offload_manager",
    "init",
    "load_config",
    "load_config_from_env",
    "load_config_from_file",
    "load_model_from_profile",
    "load_profile",
    "load_state",
    "offload",
    "offload_block",
    "offload_from_profile",
    "offload_from_state",
    "offload_units",
    "pause_profiling",
    "release",
    "request_strategy_replan",
    "reset_offload_timing",
    "resident_units",
    "resume_profiling",
    "save_profile",
    "save_state",
    "set_config",
    "suspend_profiling",
    "update_offload_timing",
    "update_state",
]
