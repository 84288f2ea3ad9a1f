"""Saved offload profiles: ``<dir>/profile.json``, schema version 3.

Same field names, JSON shape and consistency rules as the reference's
``TensorManagerState`` (state_handler.py:162-480), so a profile written by one
side can be read by the other:

* tensor ids are process-local; ``tensor_id_to_name_map`` ties each to a
  parameter name, and loading re-binds by name;
* ``load_strategy`` maps each transfer label to the tensors it streams;
* ``allocation_ordered`` / ``label_to_block_id`` / ``block_sizes`` /
  ``transfer_to_compute_map`` are the slot plan (``BlockStrategyData``);
* ``view_tensors_*`` are the streamed tensors, ``gpu_tensors_names`` the ones
  placed on the GPU for good.

A profile lets :func:`~flextensor_amd.manager.offload_from_profile` skip the
discovery and profiling passes.
"""

from __future__ import annotations

import json
import os
import struct
import tempfile
from collections import Counter
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, ClassVar

import torch

from .layout import is_packed_layout
from .planner import BlockStrategyData, LayerStatistics, TensorStatistics

PROFILE_FILE = "profile.json"
LOADER_TYPES = ("allocation_block_transfer", "raw_block_transfer", "strategy")


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _ts_dict(t: TensorStatistics) -> dict[str, Any]:
    return {"tensor_id": t.tensor_id, "name": t.name, "size_bytes": t.size_bytes, "load_time_ms": t.load_time_ms}


@dataclass
class TensorManagerState:
    SCHEMA_VERSION: ClassVar[int] = 3

    loader_type: str
    tensor_id_to_name_map: dict[int, str]
    allocation_ordered: dict[int, list[str]]
    label_to_size_map: dict[str, int]
    block_sizes: dict[int, int]
    load_strategy: dict[str, list[TensorStatistics]]
    release_strategy: dict[str, list[TensorStatistics]]
    label_to_block_id: dict[str, int]
    stats: list[LayerStatistics]
    transfer_to_compute_map: dict[str, str]
    view_tensors_ids: list[int]
    view_tensors_names: list[str]
    gpu_tensors_names: list[str]
    shm_block_name_map: dict[str, str] | None = None
    managed_tensor_dtypes: dict[str, str] = field(default_factory=dict)
    managed_tensor_layouts: dict[str, dict[str, list[int]]] = field(default_factory=dict)
    # The copy-engine policy chosen from the measured link when the plan was made (this build's addition:
    # readers that do not know the key ignore it, as the reference's reader does; None when absent).
    copy_policy: dict[str, Any] | None = None

    # ---- consistency --------------------------------------------------------

    def validate_internal(self) -> None:
        """Checks that need no live model (state_handler.py:197-338)."""

        def bad(detail: str) -> ValueError:
            return ValueError(f"Saved state mismatch: {detail}. Re-profile the model.")

        if self.loader_type not in LOADER_TYPES:
            raise ValueError(f"Unknown loader type: {self.loader_type}")
        names = list(self.tensor_id_to_name_map.values())
        dups = sorted(n for n, c in Counter(names).items() if c > 1)
        if dups:
            raise bad(f"tensor_id_to_name_map inventory names must be unique; duplicates={dups}")
        every = [t for ts in self.load_strategy.values() for t in ts]
        every += [t for ts in self.release_strategy.values() for t in ts]
        every += [t for layer in self.stats for t in layer.tensors]
        for t in every:
            if self.tensor_id_to_name_map.get(t.tensor_id) != t.name:
                raise bad(f"TensorStatistics tensor_id/name pair disagrees with tensor_id_to_name_map: "
                          f"tensor_id={t.tensor_id}, name={t.name!r}")
        if len(self.view_tensors_ids) != len(self.view_tensors_names):
            raise bad("view_tensors_ids and view_tensors_names must have equal lengths")
        if len(set(self.view_tensors_ids)) != len(self.view_tensors_ids) or \
                len(set(self.view_tensors_names)) != len(self.view_tensors_names):
            raise bad("view_tensors_ids and view_tensors_names must each be unique")
        for tid, name in zip(self.view_tensors_ids, self.view_tensors_names):
            if self.tensor_id_to_name_map.get(tid) != name:
                raise bad(f"view_tensors_ids/view_tensors_names pair disagrees with tensor_id_to_name_map: "
                          f"tensor_id={tid}, name={name!r}")
        known = set(names)
        referenced = {t.name for t in every} | set(self.view_tensors_names) | set(self.gpu_tensors_names)
        if referenced - known:
            raise bad(f"state references names outside saved inventory: {sorted(referenced - known)}")
        managed = {t.name for ts in self.load_strategy.values() for t in ts} | set(self.view_tensors_names)
        for kind, table in (("managed_tensor_dtypes", self.managed_tensor_dtypes),
                            ("managed_tensor_layouts", self.managed_tensor_layouts)):
            if table and set(table) != managed:
                raise bad(f"{kind} must be empty for a legacy profile or cover every managed tensor: "
                          f"missing={sorted(managed - set(table))}, unexpected={sorted(set(table) - managed)}")
        for name, dt in self.managed_tensor_dtypes.items():
            parsed = getattr(torch, dt, None) if isinstance(dt, str) and dt else None
            if not isinstance(parsed, torch.dtype) or _dtype_name(parsed) != dt:
                raise bad(f"invalid dtype metadata for {name!r}: {dt!r}")
        for name, lay in self.managed_tensor_layouts.items():
            if not isinstance(lay, dict) or set(lay) != {"shape", "stride"}:
                raise bad(f"invalid layout metadata for {name!r}: expected shape and stride")
            shape, stride = lay["shape"], lay["stride"]
            if not isinstance(shape, list) or not isinstance(stride, list) or len(shape) != len(stride) or \
                    any(type(x) is not int or x < 0 for x in [*shape, *stride]):
                raise bad(f"invalid layout metadata for {name!r}: shape and stride must be equal-length lists of "
                          "non-negative integers")
            if not is_packed_layout(shape, stride):
                raise bad(f"invalid layout metadata for {name!r}: tensor layout must be non-overlapping and dense")
            try:  # sizes and strides torch can represent (utils.py:101-111, state_handler.py:271-276)
                torch.empty_strided(shape, stride, device="meta")
            except (RuntimeError, OverflowError, TypeError, ValueError) as exc:
                raise bad(f"invalid layout metadata for {name!r}: {exc}") from exc
        if set(self.gpu_tensors_names) != known - managed:
            raise bad("gpu_tensors_names does not match computed final-GPU inventory: "
                      f"missing={sorted((known - managed) - set(self.gpu_tensors_names))}, "
                      f"unexpected={sorted(set(self.gpu_tensors_names) - (known - managed))}")
        if self.loader_type == "strategy":
            return
        load = {label: ts for label, ts in self.load_strategy.items() if ts}
        owners: dict[str, set[str]] = {}
        for label, ts in load.items():
            for n in {t.name for t in ts}:
                owners.setdefault(n, set()).add(label)
        multi = {n: sorted(ls) for n, ls in owners.items() if len(ls) > 1}
        if multi:
            raise bad(f"tensor names cannot belong to multiple nonempty block load labels: {multi}")
        if set(self.view_tensors_names) != set(owners):
            raise bad("view_tensors_names must match names owned by block load_strategy")
        placed = [label for labels in self.allocation_ordered.values() for label in labels]
        counts = Counter(placed)
        if set(counts) != set(load) or any(c != 1 for c in counts.values()) or \
                any(not labels for labels in self.allocation_ordered.values()):
            raise bad("allocation_ordered must contain every nonempty load label exactly once")
        if self.label_to_block_id != {label: b for b, labels in self.allocation_ordered.items() for label in labels}:
            raise bad("label_to_block_id disagrees with allocation_ordered")
        sizes = {label: sum(t.size_bytes for t in ts) for label, ts in load.items()}
        if self.label_to_size_map and self.label_to_size_map != sizes:
            raise bad("label_to_size_map does not match logical load-strategy sizes")
        if self.block_sizes != {b: max(sizes[label] for label in labels) for b, labels in self.allocation_ordered.items()}:
            raise bad("block_sizes do not match logical allocation_ordered capacities")
        stat_labels = {layer.label for layer in self.stats}
        if set(self.transfer_to_compute_map) != set(load) or set(self.transfer_to_compute_map.values()) - stat_labels:
            raise bad("transfer_to_compute_map must cover the load labels and reference known stats labels")

    # ---- JSON -----------------------------------------------------------------

    def to_dict(self) -> dict[str, Any]:
        return {
            "version": self.SCHEMA_VERSION,
            "loader_type": self.loader_type,
            "tensor_id_to_name_map": {str(k): v for k, v in self.tensor_id_to_name_map.items()},
            "allocation_ordered": {str(k): v for k, v in self.allocation_ordered.items()},
            "label_to_size_map": dict(self.label_to_size_map),
            "block_sizes": {str(k): v for k, v in self.block_sizes.items()},
            "load_strategy": {k: [_ts_dict(t) for t in v] for k, v in self.load_strategy.items()},
            "release_strategy": {k: [_ts_dict(t) for t in v] for k, v in self.release_strategy.items()},
            "label_to_block_id": dict(self.label_to_block_id),
            "stats": [{"label": s.label, "tensors": [_ts_dict(t) for t in s.tensors], "duration": s.duration}
                      for s in self.stats],
            "transfer_to_compute_map": dict(self.transfer_to_compute_map),
            "view_tensors_ids": list(self.view_tensors_ids),
            "view_tensors_names": list(self.view_tensors_names),
            "gpu_tensors_names": list(self.gpu_tensors_names),
            "shm_block_name_map": self.shm_block_name_map,
            "managed_tensor_dtypes": dict(self.managed_tensor_dtypes),
            "managed_tensor_layouts": {k: dict(v) for k, v in self.managed_tensor_layouts.items()},
            **({"copy_policy": dict(self.copy_policy)} if self.copy_policy is not None else {}),
        }

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "TensorManagerState":
        version = data.get("version", 1)
        if version > cls.SCHEMA_VERSION:
            raise ValueError(f"State file schema version {version} is newer than supported version "
                             f"{cls.SCHEMA_VERSION}.")
        if version < cls.SCHEMA_VERSION:
            raise ValueError(f"State file schema version {version} is outdated (current: {cls.SCHEMA_VERSION}). "
                             "Re-run profiling to generate a new profile.")

        def ts(d: dict[str, Any]) -> TensorStatistics:
            return TensorStatistics(int(d["tensor_id"]), d["name"], int(d["size_bytes"]), float(d["load_time_ms"]))

        state = cls(
            loader_type=data["loader_type"],
            tensor_id_to_name_map={int(k): v for k, v in data["tensor_id_to_name_map"].items()},
            allocation_ordered={int(k): list(v) for k, v in data["allocation_ordered"].items()},
            label_to_size_map={str(k): int(v) for k, v in data["label_to_size_map"].items()},
            block_sizes={int(k): int(v) for k, v in data["block_sizes"].items()},
            load_strategy={k: [ts(t) for t in v] for k, v in data["load_strategy"].items()},
            release_strategy={k: [ts(t) for t in v] for k, v in data["release_strategy"].items()},
            label_to_block_id={k: int(v) for k, v in data["label_to_block_id"].items()},
            stats=[LayerStatistics(s["label"], [ts(t) for t in s["tensors"]], float(s["duration"]))
                   for s in data["stats"]],
            transfer_to_compute_map=dict(data["transfer_to_compute_map"]),
            view_tensors_ids=[int(x) for x in data["view_tensors_ids"]],
            view_tensors_names=list(data["view_tensors_names"]),
            gpu_tensors_names=list(data["gpu_tensors_names"]),
            shm_block_name_map=data.get("shm_block_name_map"),
            managed_tensor_dtypes=dict(data.get("managed_tensor_dtypes", {})),
            managed_tensor_layouts={k: dict(v) for k, v in data.get("managed_tensor_layouts", {}).items()},
            copy_policy=dict(data["copy_policy"]) if isinstance(data.get("copy_policy"), dict) else None,
        )
        state.validate_internal()
        return state

    def block_data(self) -> BlockStrategyData:
        return BlockStrategyData(
            label_to_size_map=dict(self.label_to_size_map),
            allocation_ordered={b: list(v) for b, v in self.allocation_ordered.items()},
            block_sizes=dict(self.block_sizes),
            label_to_block_id=dict(self.label_to_block_id),
            transfer_to_compute_map=dict(self.transfer_to_compute_map),
        )


def save_state(state: TensorManagerState, directory: str | os.PathLike) -> Path:
    """Write ``<directory>/profile.json`` atomically: temporary file, then rename (state_handler.py:1422-1433)."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    target = d / PROFILE_FILE
    fd, tmp = tempfile.mkstemp(dir=d, prefix=".profile.", suffix=".tmp")
    try:
        with os.fdopen(fd, "w") as fh:
            json.dump(state.to_dict(), fh, indent=1)
        os.replace(tmp, target)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise
    return target


def _from_json_object(data: Any) -> TensorManagerState:
    if not isinstance(data, dict):
        raise ValueError("Saved state must be a JSON object")
    try:
        return TensorManagerState.from_dict(data)
    except (AttributeError, TypeError) as exc:
        raise ValueError("Saved state contains malformed nested data") from exc


def load_state(directory: str | os.PathLike) -> TensorManagerState:
    """Read and validate ``<directory>/profile.json`` (state_handler.py:1436-1454)."""
    path = Path(directory) / PROFILE_FILE
    if not path.exists():
        raise FileNotFoundError(f"no {PROFILE_FILE} in {directory}")
    return _from_json_object(json.loads(path.read_text()))


def save_state_to_bytes(state: TensorManagerState) -> bytes:
    """Big-endian u32 length, then compact JSON (state_handler.py:1457-1471)."""
    payload = json.dumps(state.to_dict(), separators=(",", ":")).encode("utf-8")
    return struct.pack("!I", len(payload)) + payload


def load_state_from_bytes(data: bytes | bytearray | memoryview) -> TensorManagerState:
    """Inverse of :func:`save_state_to_bytes`; short buffers raise ``ValueError`` (state_handler.py:1474-1500)."""
    if len(data) < 4:
        raise ValueError(f"Buffer too short: expected at least 4 bytes for length prefix, got {len(data)}")
    length = struct.unpack("!I", bytes(data[:4]))[0]
    if len(data) < 4 + length:
        raise ValueError(f"Buffer too short: length prefix indicates {length} bytes, "
                         f"but only {len(data) - 4} bytes available after prefix")
    return _from_json_object(json.loads(bytes(data[4:4 + length])))
