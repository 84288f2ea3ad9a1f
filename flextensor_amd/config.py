"""``OffloadConfig``: the reference's field names and defaults for this path.

Kept from config.py:55-402: ``enabled``, ``gpu_device``, ``pinned_memory``,
``pinned_memory_mode``, ``discovery_iters``, ``profiling_iters``,
``transfer_mode``, ``num_blocks``, ``min_blocks``, ``max_gpu_mem_fraction``,
``offload_timing``, ``piecewise_prefetch``, ``include_patterns``,
``exclude_patterns``, ``profile_storage_dir``. :func:`load_config`,
:func:`load_config_from_file` and :func:`load_config_from_env` read INI, JSON
or YAML files and ``FT_*`` environment variables with the reference's
precedence and text conversions (config.py:560-1060).

Also kept: ``shm_enabled``, ``shm_namespace``, ``shm_wait_timeout``
(config.py:97-125), ``skip_discovery`` (:133-160), ``profile_read_only``
(:240-241) and ``enable_diagnostics`` (:377-380).

Accepted for compatibility, acting differently or not at all here:

* ``external_compile`` (:172-191): the ``flextensor::pre_compute`` /
  ``post_compute`` ops are always in place, so a caller may compile each unit
  after INFERENCE without it.
* ``profile_mode`` (:382-402): profiling here always loads a unit's tensors
  on entry. ``"view"`` and ``"getter"`` both select that;
  ``"torch_function"`` needs the per-tensor strategy loader and is refused.
* ``load_strategy`` (:243-244), ``transfer_budget_scale`` (:193-200),
  ``enable_instrumentation`` and ``instrumentation_output_dir``
  (:246-250): they steer the strategy search and the instrumentation
  subsystem, which are not part of this build. A value other than the
  default logs a warning at ``offload()``.

Added for this build: ``max_gpu_mem_bytes`` (a budget in bytes instead of a
fraction), ``copy_engine`` (``auto`` / ``sdma`` / ``kernel`` / ``staged``),
``loader_order`` (``auto`` / ``default`` / ``reordered``),
``max_inflight_passes`` (bounded host run-ahead), ``encode_streamed_blocks``
(streamed blocks cross the link exponent-coded and are decoded on the GPU) and
``encode_resident_blocks`` (resident units kept exponent-coded in HBM, so more
of them fit the budget and fewer stream).
"""

from __future__ import annotations

import configparser
import difflib
import json
import os
import types
import typing
from pathlib import Path
from typing import Any, Literal

import yaml

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
    # With copy_engine="auto", time both copy engines on this device at the INFERENCE transition and
    # choose the engine per chunk size from the measured curves (the role of the reference's live
    # transfer benchmark, memory_transfer_benchmark.py:59-129). False keeps the library's default policy.
    link_benchmark: bool = True
    loader_order: Literal["auto", "default", "reordered"] = "auto"
    # Before the host enqueues a streamed forward it waits until the forward
    # this many passes back has finished on the device (0: never waits). A host
    # that runs further ahead fills the device command queue and then issues
    # each next transfer late, which idles the host link.
    max_inflight_passes: int = Field(default=1, ge=0)
    # Carry each streamed block over the link exponent-coded (about 0.75 of its bytes for bf16 weights)
    # and decode it into its ring slot with a zero-copy kernel; the slot receives the raw bytes exactly.
    # A block is kept encoded only when that saves a tenth of its bytes. allocation_block_transfer only.
    encode_streamed_blocks: bool = False
    # When the resident units do not fit the GPU budget raw, keep some exponent-coded in device memory
    # (about 0.75 of their bytes) instead of streaming more units; each such unit is decoded from HBM into
    # one shared slot on the compute stream as it runs. For link-bound passes: the fewer units stream, the
    # fewer bytes cross the link. allocation_block_transfer only, without shm_enabled.
    encode_resident_blocks: bool = False
    # Cross-process sharing of the streamed blocks through POSIX shared memory
    # (config.py:97-125): blocks live in named segments under ``shm_namespace``.
    shm_enabled: bool = False
    shm_namespace: str | None = None
    shm_wait_timeout: float = Field(default=0.0, ge=0.0)
    skip_discovery: bool = False
    profile_read_only: bool = False
    enable_diagnostics: bool = False
    external_compile: bool = False
    profile_mode: Literal["view", "getter", "torch_function"] = "view"
    load_strategy: Any = None
    transfer_budget_scale: float = Field(default=1.0, gt=0.0)
    enable_instrumentation: bool = False
    instrumentation_output_dir: str = ".flextensor/instrumentation"

    @model_validator(mode="after")
    def _check(self) -> "OffloadConfig":
        if self.transfer_mode not in TRANSFER_MODES:
            raise ValueError(f"transfer_mode must be one of {TRANSFER_MODES}, got {self.transfer_mode!r}")
        if self.shm_enabled and (self.shm_namespace is None or not self.shm_namespace.strip()):
            raise ValueError("shm_namespace must be non-empty when shm_enabled=True")
        if self.encode_streamed_blocks and self.transfer_mode != "allocation_block_transfer":
            raise ValueError("encode_streamed_blocks needs transfer_mode='allocation_block_transfer'")
        if self.encode_resident_blocks and self.transfer_mode != "allocation_block_transfer":
            raise ValueError("encode_resident_blocks needs transfer_mode='allocation_block_transfer'")
        if self.encode_resident_blocks and self.shm_enabled:
            raise ValueError("encode_resident_blocks keeps its host blocks private: it cannot be combined with "
                             "shm_enabled")
        if self.num_blocks < self.min_blocks:
            raise ValueError(f"num_blocks ({self.num_blocks}) must be >= min_blocks ({self.min_blocks})")
        if self.profile_mode == "torch_function":
            raise ValueError("profile_mode='torch_function' is only valid with transfer_mode='strategy', which this "
                             f"build does not provide; use 'view' or 'getter' with {self.transfer_mode!r}")
        return self

    def inert_settings(self) -> list[str]:
        """Settings given a non-default value that this build does not act on."""
        inert = []
        if self.load_strategy is not None:
            inert.append("load_strategy")
        if self.transfer_budget_scale != 1.0:
            inert.append("transfer_budget_scale")
        if self.enable_instrumentation:
            inert.append("enable_instrumentation")
        return inert


PinnedMemoryMode = Literal["torch", "host_register"]


# ---- loading from files and the environment (config.py:560-1060) ------------------


def _field_kind(annotation: Any) -> type:
    """The conversion type of a field: bool/int/float/str, list, or object (not loadable from text)."""
    if annotation is None:
        return str
    origin = typing.get_origin(annotation)
    if origin in (typing.Union, types.UnionType):
        kinds = [_field_kind(a) for a in typing.get_args(annotation) if a is not type(None)]
        return kinds[0] if kinds else str
    if origin is list:
        return list
    if origin is Literal:
        first = typing.get_args(annotation)[0] if typing.get_args(annotation) else ""
        return type(first) if type(first) in (bool, int, float, str) else str
    if annotation in (bool, int, float, str):
        return annotation
    return object


def _field_kinds() -> dict[str, type]:
    return {name: _field_kind(f.annotation) for name, f in OffloadConfig.model_fields.items()}


def _parse_bool(value: str) -> bool:
    low = value.lower()
    if low in ("true", "1", "yes", "y", "on"):
        return True
    if low in ("false", "0", "no", "n", "off"):
        return False
    raise ValueError(f"Cannot parse '{value}' as boolean")


def _convert(value: str, kind: type) -> Any:
    """Text -> field value: ``none``/``null``/empty is None, then by the field's type."""
    if value == "" or value.lower() in ("none", "null"):
        return None
    if kind is bool:
        return _parse_bool(value)
    if kind is int:
        return int(value)
    if kind is float:
        return float(value)
    return value


def _split_list(value: str) -> list[str]:
    return [p.strip() for p in value.split(",") if p.strip()]


def _from_mapping(data: dict[str, Any], kinds: dict[str, type]) -> dict[str, Any]:
    out: dict[str, Any] = {}
    for name, value in data.items():
        kind = kinds.get(name)
        if kind is None or kind is object:
            continue
        if kind is not list and kind is not str and isinstance(value, str):
            out[name] = _convert(value, kind)
        else:
            out[name] = value
    return out


def _load_file(path: Path, kinds: dict[str, type]) -> dict[str, Any]:
    suffix = path.suffix.lower()
    if suffix in (".conf", ".ini"):
        parser = configparser.ConfigParser()
        parser.read(path)
        if "flextensor" not in parser:
            raise ValueError("INI file must contain [flextensor] section")
        sec = parser["flextensor"]
        out: dict[str, Any] = {}
        for name, kind in kinds.items():
            if name in sec and kind is not object:
                out[name] = _split_list(sec[name]) if kind is list else _convert(sec[name], kind)
        return out
    if suffix == ".json":
        with path.open() as fh:
            data = json.load(fh)
    elif suffix in (".yaml", ".yml"):
        with path.open() as fh:
            data = yaml.safe_load(fh) or {}
    else:
        raise ValueError(f"Unsupported config file format: {suffix}. Use .conf, .ini, .json, .yaml, or .yml")
    if not isinstance(data, dict):
        raise ValueError(f"config file {path} must hold a mapping")
    return _from_mapping(data, kinds)


def _load_env(prefix: str, kinds: dict[str, type], config_file_env_var: str) -> dict[str, Any]:
    if prefix:
        known = {f"{prefix}{n.upper()}" for n in kinds} | {f"{prefix}CONFIG_FILE"}
        if config_file_env_var:
            known.add(config_file_env_var)
        errors = []
        for var in sorted(v for v in os.environ if v.startswith(prefix) and v not in known):
            msg = f"Unrecognized environment variable with {prefix} prefix: {var}"
            close = difflib.get_close_matches(var, sorted(known), n=1, cutoff=0.75)
            errors.append(msg + (f". Did you mean: {close[0]}?" if close else ""))
        if errors:
            raise ValueError("\n".join(errors))
    out: dict[str, Any] = {}
    for name, kind in kinds.items():
        if kind is object:
            continue
        var = f"{prefix}{name.upper()}"
        raw = os.environ.get(var)
        if raw is None:
            continue
        try:
            out[name] = _split_list(raw) if kind is list else _convert(raw, kind)
        except (ValueError, TypeError) as exc:
            raise ValueError(f"Failed to convert {var}={raw}: {exc}") from exc
    return out


def load_config(config_path: str | os.PathLike | None = None, env_prefix: str = "FT_", use_env: bool = True,
                config_file_env_var: str = "FT_CONFIG_FILE", **kwargs: Any) -> OffloadConfig:
    """``OffloadConfig`` from a file, then ``FT_*`` variables, then ``kwargs`` (config.py:900-969).

    Files: INI (``.conf``/``.ini``, section ``[flextensor]``), JSON or YAML.
    With no file, ``enabled`` defaults to False: offloading from the
    environment alone needs ``FT_ENABLED=1``. List fields take
    comma-separated text; ``none``/``null`` is None; booleans accept
    true/false, 1/0, yes/no, y/n, on/off.
    """
    kinds = _field_kinds()
    data: dict[str, Any] = {}
    path = config_path if config_path is not None else (os.environ.get(config_file_env_var)
                                                         if config_file_env_var else None)
    if path is not None:
        p = Path(path)
        if not p.exists():
            raise FileNotFoundError(f"Config file not found: {p}")
        data = _load_file(p, kinds)
    elif use_env:
        data["enabled"] = False
    if use_env:
        data.update(_load_env(env_prefix, kinds, config_file_env_var))
    data.update(kwargs)
    return OffloadConfig(**data)


def load_config_from_file(config_path: str | os.PathLike | None = None, env_var: str = "FT_CONFIG_FILE",
                          **kwargs: Any) -> OffloadConfig:
    """File values, then ``kwargs``; no environment overrides (config.py:972-1009)."""
    if config_path is None and os.environ.get(env_var) is None:
        raise FileNotFoundError(f"No config file specified. Provide config_path or set {env_var} environment variable.")
    return load_config(config_path=config_path, use_env=False, config_file_env_var=env_var, **kwargs)


def load_config_from_env(prefix: str = "FT_", **kwargs: Any) -> OffloadConfig:
    """``<prefix><FIELD>`` variables, then ``kwargs``; ``enabled`` defaults to False (config.py:1012-1059)."""
    return load_config(config_path=None, env_prefix=prefix, use_env=True, config_file_env_var="", **kwargs)
