"""Build a model from a saved profile and a safetensors checkpoint without a full host copy.

The reference's ``load_model_from_profile`` (lazy_model_init.py:500-604)
constructs the model with parameters on the meta device and buffers on the
GPU, reads the profile's resident and streamed tensors out of the checkpoint,
assigns them and adopts the saved plan. This module keeps that interface and
changes how the bytes travel:

* **The checkpoint is mapped, not read.** :class:`SafetensorsFile` parses the
  safetensors header itself and hands out tensors that are zero-copy views of a
  private file mapping. The streamed weights then go from the page cache
  straight into their packed page-locked blocks (one host copy; the reference
  reads each tensor into a fresh host tensor and packs it, two copies), and the
  resident weights straight to HBM through the library's staged copy engine.
  For a 70B fp8 checkpoint that is 68 GB of host copying and 68 GB of peak
  host memory saved.
* **Construction costs no parameter memory.** While the model class runs,
  every parameter it registers is moved to the meta device (its values are
  never read), every buffer to ``buffer_device``. The patch of
  ``nn.Module.register_parameter`` / ``register_buffer`` acts only on the
  thread that is constructing; other threads see the original behaviour.
* **Object identity is kept.** Parameters are replaced object for object
  across the model: tied weights stay tied and attributes that point at a
  parameter (``self.weight.scale = self.scale = nn.Parameter(...)``, the
  pattern of DeepSeek-V3-style fp8 layers) follow the replacement, both when
  construction swaps a parameter for its meta twin and when loading swaps the
  meta twin for the checkpoint tensor. The reference tracks these links by name
  on a second, meta-device construction (lazy_model_init.py:227-470); here the
  one construction records the swaps it makes.

The safetensors format (an 8-byte little-endian header length, a JSON header
of ``{name: {dtype, shape, data_offsets}}`` plus optional ``__metadata__``,
then the raw little-endian tensor bytes) is the published format of the
``safetensors`` package; the parser here is this package's own.
"""
from __future__ import annotations

import contextlib
import json
import logging
import math
import mmap
import os
import struct
import threading
from collections.abc import Iterable, Iterator, Mapping
from typing import Any

import torch
from torch import nn

from .config import OffloadConfig
from .profile import load_state

LOGGER = logging.getLogger(__name__)

__all__ = [
    "SafetensorsFile",
    "create_split_device_model",
    "load_model_from_profile",
    "load_specific_keys",
    "split_device_init",
]

_BLOCK_LOADERS = ("allocation_block_transfer", "raw_block_transfer")
_MAX_HEADER_BYTES = 100 * 1024 * 1024

_DTYPES: dict[str, torch.dtype] = {
    "F64": torch.float64,
    "F32": torch.float32,
    "F16": torch.float16,
    "BF16": torch.bfloat16,
    "F8_E4M3": torch.float8_e4m3fn,
    "F8_E5M2": torch.float8_e5m2,
    "I64": torch.int64,
    "I32": torch.int32,
    "I16": torch.int16,
    "I8": torch.int8,
    "U64": torch.uint64,
    "U32": torch.uint32,
    "U16": torch.uint16,
    "U8": torch.uint8,
    "BOOL": torch.bool,
}


class SafetensorsFile:
    """A safetensors checkpoint mapped into memory; :meth:`get` returns zero-copy host tensors.

    The file is mapped privately (copy-on-write): a tensor may be written to
    without changing the file. The mapping lives as long as the last tensor
    that views it, so there is no ``close``; dropping the object and every
    tensor taken from it releases the mapping.
    """

    def __init__(self, path: str | os.PathLike[str]) -> None:
        self.path = os.fspath(path)
        size = os.path.getsize(self.path)
        with open(self.path, "rb") as f:
            head = f.read(8)
            if len(head) < 8:
                raise ValueError(f"{self.path}: not a safetensors file (shorter than its 8-byte header length)")
            (header_len,) = struct.unpack("<Q", head)
            if header_len > min(_MAX_HEADER_BYTES, size - 8):
                raise ValueError(f"{self.path}: header length {header_len} does not fit the file of {size} bytes")
            try:
                header = json.loads(f.read(header_len))
            except (UnicodeDecodeError, json.JSONDecodeError) as exc:
                raise ValueError(f"{self.path}: the header is not valid JSON: {exc}") from None
            if not isinstance(header, dict):
                raise ValueError(f"{self.path}: the header is not a JSON object")
            self.metadata: dict[str, str] = dict(header.pop("__metadata__", None) or {})
            self._data_start = 8 + header_len
            data_bytes = size - self._data_start
            self._entries: dict[str, tuple[torch.dtype, tuple[int, ...], int, int]] = {}
            for name, e in header.items():
                self._entries[name] = self._check_entry(name, e, data_bytes)
            self._map = (mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_COPY) if size > 0 else None)

    def _check_entry(self, name: str, e: Any, data_bytes: int) -> tuple[torch.dtype, tuple[int, ...], int, int]:
        try:
            dtype = _DTYPES[e["dtype"]]
            shape = tuple(int(x) for x in e["shape"])
            begin, end = (int(x) for x in e["data_offsets"])
        except (KeyError, TypeError, ValueError):
            raise ValueError(f"{self.path}: tensor {name!r} has a malformed or unsupported entry {e!r}") from None
        nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
        if any(x < 0 for x in shape) or not 0 <= begin <= end <= data_bytes or end - begin != nbytes:
            raise ValueError(f"{self.path}: tensor {name!r} ({e['dtype']} {list(shape)}) has offsets "
                             f"[{begin}, {end}) that do not hold {nbytes} bytes inside the {data_bytes}-byte data")
        return dtype, shape, begin, end

    def keys(self) -> list[str]:
        return list(self._entries)

    def __contains__(self, name: object) -> bool:
        return name in self._entries

    def __len__(self) -> int:
        return len(self._entries)

    def dtype(self, name: str) -> torch.dtype:
        return self._entries[name][0]

    def shape(self, name: str) -> tuple[int, ...]:
        return self._entries[name][1]

    def get(self, name: str) -> torch.Tensor:
        """The tensor ``name`` as a C-contiguous host tensor over the mapped file (no copy)."""
        try:
            dtype, shape, begin, end = self._entries[name]
        except KeyError:
            raise KeyError(f"{name!r} is not in {self.path}") from None
        if begin == end:
            return torch.empty(shape, dtype=dtype)
        flat = torch.frombuffer(self._map, dtype=torch.uint8, count=end - begin, offset=self._data_start + begin)
        return flat.view(dtype).view(shape)

    def tensors(self, names: Iterable[str], *, strict: bool = False) -> dict[str, torch.Tensor]:
        """``{name: tensor}`` for the requested names present in the file.

        With ``strict`` a missing name raises ``KeyError`` listing every
        missing name; otherwise missing names are left out.
        """
        names = list(names)
        if strict:
            missing = [n for n in names if n not in self._entries]
            if missing:
                raise KeyError(f"Missing keys in safetensors file '{self.path}': {missing}")
        return {n: self.get(n) for n in names if n in self._entries}


def load_specific_keys(file_path: str | os.PathLike[str], keys: list[str], device: str | torch.device = "cpu", *,
                       strict: bool = False) -> dict[str, torch.Tensor]:
    """Only the named tensors of a safetensors file (lazy_model_init.py:22-55).

    On ``"cpu"`` the tensors are zero-copy views of the mapped file; on any
    other device they are copied there. ``strict`` raises ``KeyError`` for
    missing keys, otherwise they are skipped.
    """
    found = SafetensorsFile(file_path).tensors(keys, strict=strict)
    dev = torch.device(device)
    if dev.type == "cpu":
        return found
    return {n: t.to(dev) for n, t in found.items()}


# -- split-device construction ---------------------------------------------------------------------

class _SplitInit:
    def __init__(self, param_device: torch.device, buffer_device: torch.device) -> None:
        self.param_device = param_device
        self.buffer_device = buffer_device
        self.swapped: dict[int, tuple[nn.Parameter, nn.Parameter]] = {}


_TLS = threading.local()
_PATCH_LOCK = threading.Lock()
_PATCH_USERS = 0
_ORIGINAL: dict[str, Any] = {}


def _patched_register_parameter(self: nn.Module, name: str, param: nn.Parameter | None) -> None:
    ctx: _SplitInit | None = getattr(_TLS, "ctx", None)
    if ctx is not None and param is not None and param.device != ctx.param_device:
        twin = nn.Parameter(param.detach().to(ctx.param_device), requires_grad=param.requires_grad)
        twin.__dict__.update(param.__dict__)
        ctx.swapped[id(param)] = (param, twin)
        param.data = torch.empty(0, dtype=param.dtype, device=param.device)  # the values are never read
        param = twin
    _ORIGINAL["register_parameter"](self, name, param)


def _patched_register_buffer(self: nn.Module, name: str, tensor: torch.Tensor | None, persistent: bool = True) -> None:
    ctx: _SplitInit | None = getattr(_TLS, "ctx", None)
    if ctx is not None and tensor is not None and tensor.device != ctx.buffer_device and tensor.device.type != "meta":
        tensor = tensor.to(ctx.buffer_device)  # a buffer made from a meta parameter stays meta
    _ORIGINAL["register_buffer"](self, name, tensor, persistent=persistent)


def _canonical(device: str | torch.device) -> torch.device:
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


@contextlib.contextmanager
def split_device_init(param_device: str | torch.device = "meta",
                      buffer_device: str | torch.device = "cuda") -> Iterator[_SplitInit]:
    """Within the block, modules built on this thread register parameters on ``param_device``
    and buffers on ``buffer_device`` (the role of ``ModulePatcher``, lazy_model_init.py:110-180).

    The ``nn.Module`` registration methods are replaced while any thread is
    inside such a block; the replacements act only for the thread that
    entered it. Nesting on one thread is not supported.
    """
    global _PATCH_USERS
    if getattr(_TLS, "ctx", None) is not None:
        raise RuntimeError("split_device_init is already active on this thread")
    ctx = _SplitInit(_canonical(param_device), _canonical(buffer_device))
    with _PATCH_LOCK:
        if _PATCH_USERS == 0:
            _ORIGINAL["register_parameter"] = nn.Module.register_parameter
            _ORIGINAL["register_buffer"] = nn.Module.register_buffer
            nn.Module.register_parameter = _patched_register_parameter  # type: ignore[method-assign]
            nn.Module.register_buffer = _patched_register_buffer  # type: ignore[method-assign]
        _PATCH_USERS += 1
    _TLS.ctx = ctx
    try:
        yield ctx
    finally:
        _TLS.ctx = None
        with _PATCH_LOCK:
            _PATCH_USERS -= 1
            if _PATCH_USERS == 0:
                nn.Module.register_parameter = _ORIGINAL.pop("register_parameter")  # type: ignore[method-assign]
                nn.Module.register_buffer = _ORIGINAL.pop("register_buffer")  # type: ignore[method-assign]


def _replace_parameters(model: nn.Module, swaps: Mapping[int, tuple[nn.Parameter, nn.Parameter]]) -> int:
    """Put the new parameter wherever the model holds an old one; returns the slots changed.

    Covers registered slots (so tied weights stay tied) and parameter
    attributes that point at a parameter.
    """
    changed = 0
    for mod in model.modules():
        for key, p in mod._parameters.items():
            if p is not None and id(p) in swaps:
                mod._parameters[key] = swaps[id(p)][1]
                changed += 1
    for p in {id(p): p for p in model.parameters()}.values():
        for key, value in list(vars(p).items()):
            if isinstance(value, torch.Tensor) and id(value) in swaps:
                p.__dict__[key] = swaps[id(value)][1]
                changed += 1
    return changed


def create_split_device_model(model_class: type[nn.Module], model_args: tuple = (), model_kwargs: dict | None = None,
                              param_device: str | torch.device = "meta",
                              buffer_device: str | torch.device = "cuda") -> nn.Module:
    """Construct ``model_class`` with parameters on ``param_device`` and buffers on ``buffer_device``
    (lazy_model_init.py:183-224, 434-470).

    A parameter's host values are released as soon as its twin is registered,
    so constructing a model on the meta device never holds more than one
    parameter's worth of host memory. Attributes that pointed at the
    constructed parameters point at their twins afterwards.
    """
    with split_device_init(param_device, buffer_device) as ctx:
        model = model_class(*model_args, **(model_kwargs or {}))
    _replace_parameters(model, ctx.swapped)
    return model


def _assign(model: nn.Module, tensors: Mapping[str, torch.Tensor]) -> list[str]:
    """Give every parameter (and buffer) named in ``tensors`` that tensor, object for object.

    Returns the names of parameters and buffers left on the meta device.
    """
    names: dict[int, list[str]] = {}
    objs: dict[int, nn.Parameter] = {}
    for n, p in model.named_parameters(remove_duplicate=False):
        names.setdefault(id(p), []).append(n)
        objs[id(p)] = p
    swaps: dict[int, tuple[nn.Parameter, nn.Parameter]] = {}
    for tid, aliases in names.items():
        src_name = next((n for n in aliases if n in tensors), None)
        if src_name is None:
            continue
        p, src = objs[tid], tensors[src_name]
        if tuple(src.shape) != tuple(p.shape):
            raise ValueError(f"checkpoint tensor {src_name!r} has shape {list(src.shape)}, "
                             f"the model expects {list(p.shape)}")
        new = nn.Parameter(src, requires_grad=p.requires_grad and src.is_floating_point())
        new.__dict__.update(p.__dict__)
        swaps[tid] = (p, new)
    _replace_parameters(model, swaps)
    for mod_name, mod in model.named_modules(remove_duplicate=False):
        for key, b in mod._buffers.items():
            full = f"{mod_name}.{key}" if mod_name else key
            if b is not None and full in tensors:
                src = tensors[full]
                if tuple(src.shape) != tuple(b.shape):
                    raise ValueError(f"checkpoint tensor {full!r} has shape {list(src.shape)}, "
                                     f"the model expects {list(b.shape)}")
                mod._buffers[key] = src.to(b.device) if b.device.type != "meta" else src
    return [n for n, t in [*model.named_parameters(), *model.named_buffers()] if t.device.type == "meta"]


# -- the high-level loader -------------------------------------------------------------------------

def load_model_from_profile(tensor_manager: Any, profile_directory: str | os.PathLike[str],
                            model_class: type[nn.Module], model_args: tuple = (),
                            safetensor_path: str | os.PathLike[str] | None = None,
                            model_kwargs: dict | None = None, buffer_device: str | torch.device | None = None,
                            diagnose: bool = False, strict: bool = False, *,
                            config: OffloadConfig | None = None, compile_fn: Any = None) -> nn.Module:
    """Construct ``model_class`` from a saved profile and a safetensors checkpoint, ready to stream
    (lazy_model_init.py:500-604).

    ``tensor_manager`` is the :class:`~flextensor_amd.manager.OffloadManager`
    that adopts the plan (or a manager name; ``None`` is the default manager).
    The reference returns the model with the plan restored into its tensor
    manager for the caller to start; here the manager adopts the plan at once
    (the saved plan skips discovery and profiling), so the returned model
    streams on its first forward. The config is ``config``, else the manager's,
    else a default one with the profile's transfer mode.

    Only the tensors the profile names are read: ``gpu_tensors_names`` go to
    HBM, ``view_tensors_names`` into the packed page-locked blocks, both from
    the mapped file. ``strict`` raises ``KeyError`` if the file lacks any of
    them. Parameters the checkpoint does not hold would stay on the meta
    device; that raises ``RuntimeError`` naming them rather than failing in
    the first forward. ``diagnose`` logs which parameters were loaded and which
    checkpoint tensors went unused.

    Raises ``ValueError`` without ``safetensor_path`` and for a profile whose
    transfer mode is not a block mode.
    """
    from .manager import DEFAULT_MANAGER_NAME, OffloadManager, get_offload_manager

    if safetensor_path is None:
        raise ValueError("safetensor_path is required")
    if isinstance(tensor_manager, OffloadManager):
        mgr = tensor_manager
    else:
        mgr = get_offload_manager(tensor_manager if tensor_manager is not None else DEFAULT_MANAGER_NAME)
    state = load_state(profile_directory)
    if state.loader_type not in _BLOCK_LOADERS:
        raise ValueError(f"profile transfer mode {state.loader_type!r} is not one of {_BLOCK_LOADERS}")
    cfg = config or mgr.config or OffloadConfig(transfer_mode=state.loader_type)
    if buffer_device is None:
        buffer_device = torch.device("cuda", cfg.gpu_device) if torch.cuda.is_available() else torch.device("cpu")
    ckpt = SafetensorsFile(safetensor_path)
    model = create_split_device_model(model_class, model_args, model_kwargs, "meta", buffer_device).eval()
    wanted = list(dict.fromkeys([*state.gpu_tensors_names, *state.view_tensors_names]))
    tensors = ckpt.tensors(wanted, strict=strict)
    left = _assign(model, tensors)
    if diagnose:
        unused = sorted(set(ckpt.keys()) - set(tensors))
        LOGGER.info("load_model_from_profile: %d of %d profile tensors loaded from %s; %d checkpoint tensors "
                    "unused %s; still on meta: %s", len(tensors), len(wanted), ckpt.path, len(unused),
                    unused[:8], left[:8])
    if left:
        raise RuntimeError(f"{len(left)} parameters or buffers are not in the checkpoint and would stay on the meta "
                           f"device: {left[:8]}")
    return mgr.offload(model, cfg, state=state, compile_fn=compile_fn)
