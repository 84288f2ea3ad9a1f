"""``OffloadConfig``: the reference's field names and defaults for this path.

Kept from config.py:55-402: ``enabled``, ``gpu_device``, ``pinned_memory``,
``pinned_memory_mode``, ``discovery_iters``, ``profiling_iters``,
``transfer_mode``, ``num_blocks``, ``min_blocks``, ``max_gpu_mem_fraction``,
``offload_timing``, ``piecewise_prefetch``, ``include_patterns``,
``exclude_patterns``, ``profile_storage_dir``. ``FT_*`` environment variables
override fields (config.py:1012).

Also kept: ``shm_enabled``, ``shm_namespace``, ``shm_wait_timeout``
(config.py:97-125).

Added for this build: ``max_gpu_mem_bytes`` (a budget in bytes instead of a
fraction), ``copy_engine`` (``auto`` / ``sdma`` / ``kernel`` / ``staged``),
``loader_order`` (``auto`` / ``default`` / ``reordered``) and
``max_inflight_passes`` (bounded host run-ahead).
"""

from __future__ import annotations

import json
import os
from typing import Any, Literal

from pydantic import BaseModel, ConfigDict, Field, model_validator

TRANSFER_MODES = ("allocation_block_transfer", "raw_block_transfer")


class OffloadConfig(BaseModel):
    model_config = ConfigDict(extra="forbid", validate_assignment=True)

    enabled: bool = True
    gpu_device: int = Field(default=0, ge=0)
    pinned_memory: bool = True
    pinned_memory_mode: Literal["torch", "host_register"] = "torch"
    discovery_iters: int = Field(default=1, ge=0)
    profiling_iters: int = Field(default=10, ge=0)
    transfer_mode: str = "allocation_block_transfer"
    num_blocks: int = Field(default=4, ge=2)
    min_blocks: int = Field(default=4, ge=2)
    max_gpu_mem_fraction: float | None = Field(default=None, gt=0.0, le=1.0)
    max_gpu_mem_bytes: int | None = Field(default=None, gt=0)
    offload_timing: Literal["off", "eager", "cuda_graph"] = "off"
    piecewise_prefetch: Literal["off", "warn", "error"] = "warn"
    include_patterns: list[str] = Field(default_factory=lambda: ["*"])
    exclude_patterns: list[str] = Field(default_factory=list)
    profile_storage_dir: str | None = None
    copy_engine: Literal["auto", "sdma", "kernel", "staged"] = "auto"
    loader_order: Literal["auto", "default", "reordered"] = "auto"
    # Before the host enqueues a streamed forward it waits until the forward
    # this many passes back has finished on the device (0: never waits). A host
    # that runs further ahead fills the device command queue and then issues
    # each next transfer late, which idles the host link.
    max_inflight_passes: int = Field(default=1, ge=0)
    # Cross-process sharing of the streamed blocks through POSIX shared memory
    # (config.py:97-125): blocks live in named segments under ``shm_namespace``.
    shm_enabled: bool = False
    shm_namespace: str | None = None
    shm_wait_timeout: float = Field(default=0.0, ge=0.0)

    @model_validator(mode="after")
    def _check(self) -> "OffloadConfig":
        if self.transfer_mode not in TRANSFER_MODES:
            raise ValueError(f"transfer_mode must be one of {TRANSFER_MODES}, got {self.transfer_mode!r}")
        if self.shm_enabled and (self.shm_namespace is None or not self.shm_namespace.strip()):
            raise ValueError("shm_namespace must be non-empty when shm_enabled=True")
        return self


def _coerce(value: str) -> Any:
    try:
        return json.loads(value)
    except json.JSONDecodeError:
        return value


def load_config_from_env(prefix: str = "FT_", base: OffloadConfig | None = None) -> OffloadConfig:
    """``base`` (or defaults) with fields overridden by ``<prefix><FIELD>`` variables."""
    data = base.model_dump() if base is not None else {}
    for name in OffloadConfig.model_fields:
        raw = os.environ.get(prefix + name.upper())
        if raw is not None:
            data[name] = _coerce(raw)
    return OffloadConfig(**data)
