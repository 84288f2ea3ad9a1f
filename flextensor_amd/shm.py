"""Shared host memory: named segments and the resident-tensor store format.

:class:`SharedSegment` is a named POSIX shared-memory segment
(``/dev/shm/<name>``) mapped into the process. A creator fills a private
segment and then publishes it under its final name with one ``link`` call, so
a follower sees either no segment or a complete one, and a second creator of
the same name fails with ``FileExistsError`` without touching the first. The
creator's :meth:`~SharedSegment.close` removes the name; mappings already
open in other processes stay valid until they close.

:class:`SharedTensorStore` keeps the byte format of the reference's resident
tensor store (shm/tensor_store.py:33-37, 202-289, 318-412) so either side can
read a store the other wrote:

* header ``<4sIQQQ``: magic ``b"FTTS"``, version 1, manifest length, data
  offset, data size (all little endian);
* manifest: UTF-8 JSON ``{"tensors": [...]}`` with sorted keys and compact
  separators, one descriptor per unique tensor object (``aliases``,
  ``dtype``, ``kind``, ``payload_offset``, ``persistent``,
  ``requires_grad``, ``shape``, ``stride``);
* data region at a 64-byte aligned offset; each payload at an offset aligned
  to ``max(8, element size)``; a non-dense tensor is stored C-contiguous.

Materializing onto a GPU does not copy tensor by tensor as the reference
does (shm/tensor_store.py:532-569): every payload is packed chunk by chunk
into pinned staging buffers, crosses the host link in one copy per chunk and
is placed by one scatter launch per chunk (:func:`~flextensor_amd.scatter.upload_tensors`).
"""

from __future__ import annotations

import json
import math
import mmap
import os
import secrets
import struct
from collections.abc import Callable, Iterable
from dataclasses import dataclass
from itertools import pairwise
from typing import Any

import torch
from torch import nn

MAGIC = b"FTTS"
VERSION = 1
HEADER = struct.Struct("<4sIQQQ")
DATA_ALIGNMENT = 64
PAYLOAD_ALIGNMENT = 8
SHM_DIR = "/dev/shm"


def _align(value: int, alignment: int) -> int:
    return -(-value // alignment) * alignment


def store_segment_name(namespace: str) -> str:
    """Segment name of a namespace's resident tensor store (shm/tensor_store.py:45-47)."""
    return f"{namespace}_t"


# ---- segments ---------------------------------------------------------------------


class SharedSegment:
    """A named POSIX shared-memory segment mapped read-write.

    ``create=True`` with ``initializer``: the segment is created under a
    private name, ``initializer(memoryview)`` fills it, and it is published
    under ``name``. ``create=False``: an existing segment is mapped
    (``FileNotFoundError`` when absent).
    """

    def __init__(self, name: str, size: int = 0, *, create: bool = False,
                 initializer: Callable[[memoryview], None] | None = None) -> None:
        if not name or "/" in name:
            raise ValueError(f"invalid shared-memory name {name!r}")
        self.name = name
        self.path = os.path.join(SHM_DIR, name)
        self.creator = create
        self._mmap: mmap.mmap | None = None
        self._buf: memoryview | None = None
        if create:
            self._create(size, initializer)
        else:
            self._attach()

    def _map(self, fd: int, size: int) -> None:
        self._mmap = mmap.mmap(fd, size, flags=mmap.MAP_SHARED, prot=mmap.PROT_READ | mmap.PROT_WRITE)
        self._buf = memoryview(self._mmap)

    def _create(self, size: int, initializer: Callable[[memoryview], None] | None) -> None:
        if size <= 0:
            raise ValueError(f"segment size must be positive, got {size}")
        tmp = os.path.join(SHM_DIR, f".{self.name}.{secrets.token_hex(6)}")
        fd = os.open(tmp, os.O_CREAT | os.O_EXCL | os.O_RDWR, 0o600)
        try:
            os.ftruncate(fd, size)
            self._map(fd, size)
            if initializer is not None:
                # a slice of its own, dropped (not released) afterwards: tensors the initializer made
                # from it keep the mapping alive by reference
                initializer(self._buf[:])
            os.link(tmp, self.path)  # atomic publish; FileExistsError when the name is taken
        except BaseException:
            self._unmap()
            raise
        finally:
            os.close(fd)
            os.unlink(tmp)

    def _attach(self) -> None:
        fd = os.open(self.path, os.O_RDWR)
        try:
            size = os.fstat(fd).st_size
            if size == 0:
                raise RuntimeError(f"shared-memory segment {self.name!r} is empty")
            self._map(fd, size)
        finally:
            os.close(fd)

    @property
    def buf(self) -> memoryview:
        if self._buf is None:
            raise RuntimeError(f"shared-memory segment {self.name!r} is closed")
        return self._buf

    @property
    def size(self) -> int:
        return len(self.buf)

    def _unmap(self) -> None:
        """Drop this object's references to the mapping (never a forced unmap).

        ``torch.frombuffer(segment.buf)`` keeps the memoryview object alive but
        holds no buffer export, so an explicit ``mmap.close()`` would succeed
        and unmap memory that live tensors still point at. Instead the memory
        is unmapped when the last reference goes: the memoryview holds the
        mapping, and tensors hold the memoryview. With no tensor left the
        mapping goes at once (reference counting).
        """
        self._buf = None
        self._mmap = None

    def unlink(self) -> None:
        """The creator removes the name (other processes' mappings stay valid). Idempotent."""
        if self.creator:
            self.creator = False
            try:
                os.unlink(self.path)
            except FileNotFoundError:
                pass

    def close(self) -> None:
        """The creator removes the name, and this object lets go of the mapping. Idempotent.

        Safe with live tensor views: the mapping stays until the last tensor
        made from :attr:`buf` is gone, then it is unmapped.
        """
        if self._mmap is None:
            return
        self.unlink()
        self._unmap()


# ---- store format ---------------------------------------------------------------


def _is_dense(shape: tuple[int, ...], stride: tuple[int, ...]) -> bool:
    """No gaps and no overlap: sorted by stride, each stride is the product of the smaller extents."""
    if math.prod(shape) == 0:
        return True
    expect = 1
    for size, step in sorted(((n, s) for n, s in zip(shape, stride) if n > 1), key=lambda x: x[1]):
        if step != expect:
            return False
        expect *= size
    return True


def _storage_elements(shape: tuple[int, ...], stride: tuple[int, ...]) -> int:
    return 0 if math.prod(shape) == 0 else 1 + sum((n - 1) * s for n, s in zip(shape, stride))


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _parse_dtype(value: Any) -> torch.dtype:
    if not isinstance(value, str) or not value:
        raise ValueError("dtype must be a non-empty string")
    dt = getattr(torch, value, None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"unsupported dtype {value!r}")
    return dt


def _parse_layout(shape: Any, stride: Any) -> tuple[tuple[int, ...], tuple[int, ...]]:
    for field_name, v in (("shape", shape), ("stride", stride)):
        if not isinstance(v, list) or any(type(x) is not int or x < 0 for x in v):
            raise ValueError(f"{field_name} must contain non-negative integers")
    if len(shape) != len(stride):
        raise ValueError("shape/stride rank mismatch")
    if not _is_dense(tuple(shape), tuple(stride)):
        raise ValueError("tensor layout must be non-overlapping and dense")
    return tuple(shape), tuple(stride)


@dataclass(frozen=True)
class TensorDescriptor:
    """One unique parameter or buffer object in a store."""

    kind: str  # "parameter" | "buffer"
    aliases: tuple[str, ...]
    dtype: torch.dtype
    shape: tuple[int, ...]
    stride: tuple[int, ...]
    payload_offset: int
    byte_length: int
    requires_grad: bool
    persistent: tuple[bool, ...] | None

    def manifest_entry(self) -> dict[str, Any]:
        return {
            "aliases": list(self.aliases),
            "dtype": _dtype_name(self.dtype),
            "kind": self.kind,
            "payload_offset": self.payload_offset,
            "persistent": None if self.persistent is None else list(self.persistent),
            "requires_grad": self.requires_grad,
            "shape": list(self.shape),
            "stride": list(self.stride),
        }


def _owner(model: nn.Module, qualified: str) -> tuple[nn.Module, str]:
    if "." not in qualified:
        return model, qualified
    mod, leaf = qualified.rsplit(".", 1)
    return model.get_submodule(mod), leaf


def _collect(model: nn.Module, parameter_names: Iterable[str]) -> list[tuple[str, tuple[str, ...], torch.Tensor,
                                                                          tuple[bool, ...] | None]]:
    """Requested parameters (with every alias), then every registered non-None buffer, in registration order."""
    params = dict(model.named_parameters(recurse=True, remove_duplicate=False))
    buffers = dict(model.named_buffers(recurse=True, remove_duplicate=False))
    wanted = list(parameter_names)
    if any(not isinstance(n, str) or not n for n in wanted):
        raise ValueError("SharedTensorStore parameter names must be non-empty strings")
    chosen: dict[int, torch.Tensor] = {}
    for n in wanted:
        p = params.get(n)
        if p is None:
            kind = "buffer" if n in buffers else "missing"
            raise ValueError(f"SharedTensorStore requested parameter {n!r} is not a registered non-None parameter "
                             f"({kind})")
        chosen.setdefault(id(p), p)
    aliases: dict[int, list[str]] = {k: [] for k in chosen}
    for n, p in params.items():
        if id(p) in aliases:
            aliases[id(p)].append(n)
    out: list[tuple[str, tuple[str, ...], torch.Tensor, tuple[bool, ...] | None]] = [
        ("parameter", tuple(aliases[k]), p, None) for k, p in chosen.items()]
    buf_obj: dict[int, torch.Tensor] = {}
    buf_alias: dict[int, list[str]] = {}
    for n, b in buffers.items():
        buf_obj.setdefault(id(b), b)
        buf_alias.setdefault(id(b), []).append(n)
    for k, b in buf_obj.items():
        if k in chosen:
            raise ValueError("SharedTensorStore cannot encode one object as both a parameter and a buffer")
        names = tuple(buf_alias[k])
        persistent = tuple(_owner(model, n)[1] not in _owner(model, n)[0]._non_persistent_buffers_set for n in names)
        out.append(("buffer", names, b, persistent))
    return out


def plan_store(model: nn.Module, parameter_names: Iterable[str]) -> tuple[list[TensorDescriptor],
                                                                          list[torch.Tensor], bytes, int, int]:
    """Descriptors, source tensors, encoded manifest, data offset and data size of a store."""
    descs: list[TensorDescriptor] = []
    sources: list[torch.Tensor] = []
    cursor = 0
    for kind, aliases, t, persistent in _collect(model, parameter_names):
        if t.layout is not torch.strided:
            raise ValueError(f"SharedTensorStore only supports strided tensors, got {t.layout}")
        shape, stride = tuple(t.shape), tuple(t.stride())
        if any(s < 0 for s in stride):
            raise ValueError("SharedTensorStore does not support negative tensor strides")
        if not _is_dense(shape, stride):
            stride = tuple(torch.empty(shape, device="meta").stride()) if shape else ()
        nbytes = _storage_elements(shape, stride) * t.element_size()
        off = _align(cursor, max(PAYLOAD_ALIGNMENT, t.element_size()))
        descs.append(TensorDescriptor(kind, aliases, t.dtype, shape, stride, off, nbytes,
                                      bool(t.requires_grad) if kind == "parameter" else False, persistent))
        sources.append(t)
        cursor = off + nbytes
    manifest = json.dumps({"tensors": [d.manifest_entry() for d in descs]}, sort_keys=True,
                          separators=(",", ":")).encode("utf-8")
    data_offset = _align(HEADER.size + len(manifest), DATA_ALIGNMENT)
    return descs, sources, manifest, data_offset, cursor


def _payload_view(buf: memoryview, data_offset: int, d: TensorDescriptor) -> torch.Tensor:
    """A typed CPU tensor over descriptor ``d``'s payload bytes (no copy)."""
    raw = torch.frombuffer(buf, dtype=torch.uint8, count=d.byte_length, offset=data_offset + d.payload_offset)
    return torch.as_strided(raw.view(d.dtype), d.shape, d.stride, 0)


def write_store(buf: memoryview, descs: list[TensorDescriptor], sources: list[torch.Tensor], manifest: bytes,
                data_offset: int, data_size: int) -> None:
    """Header, manifest, then each source copied straight into its payload range."""
    HEADER.pack_into(buf, 0, MAGIC, VERSION, len(manifest), data_offset, data_size)
    buf[HEADER.size:HEADER.size + len(manifest)] = manifest
    for d, src in zip(descs, sources):
        if d.byte_length:
            dst = _payload_view(buf, data_offset, d)
            dst.copy_(src.detach())
            del dst


def _parse_descriptor(v: Any, data_size: int, seen: set[str]) -> TensorDescriptor:
    """One manifest entry, with the reference's checks (shm/tensor_store.py:292-380)."""
    if not isinstance(v, dict):
        raise RuntimeError("SharedTensorStore manifest tensor descriptor must be an object")
    kind = v.get("kind")
    if kind not in ("parameter", "buffer"):
        raise RuntimeError(f"SharedTensorStore manifest contains invalid tensor kind {kind!r}")
    aliases = v.get("aliases")
    if not isinstance(aliases, list) or not aliases or any(not isinstance(a, str) or not a for a in aliases):
        raise RuntimeError("SharedTensorStore manifest aliases must be non-empty strings")
    if len(set(aliases)) != len(aliases):
        raise RuntimeError("SharedTensorStore manifest aliases must be unique")
    dup = seen.intersection(aliases)
    if dup:
        raise RuntimeError(f"SharedTensorStore manifest repeats aliases {sorted(dup)!r}")
    seen.update(aliases)
    try:
        dtype = _parse_dtype(v.get("dtype"))
        shape, stride = _parse_layout(v.get("shape"), v.get("stride"))
    except ValueError as err:
        raise RuntimeError(f"SharedTensorStore manifest: {err}") from err
    off = v.get("payload_offset")
    if type(off) is not int or off < 0:
        raise RuntimeError("SharedTensorStore manifest payload offset is invalid")
    esize = torch.empty((), dtype=dtype).element_size()
    nbytes = _storage_elements(shape, stride) * esize
    if off + nbytes > data_size:
        raise RuntimeError("SharedTensorStore payload bounds exceed the declared data region")
    if off % esize:
        raise RuntimeError("SharedTensorStore payload offset is not dtype-aligned")
    rg = v.get("requires_grad")
    if not isinstance(rg, bool):
        raise RuntimeError("SharedTensorStore manifest requires_grad must be boolean")
    pers = v.get("persistent")
    if kind == "parameter":
        if pers is not None:
            raise RuntimeError("SharedTensorStore parameter descriptor cannot define buffer persistence")
        persistent = None
    else:
        if not isinstance(pers, list) or len(pers) != len(aliases) or any(not isinstance(f, bool) for f in pers):
            raise RuntimeError("SharedTensorStore buffer persistence must match its aliases")
        persistent = tuple(pers)
    return TensorDescriptor(kind, tuple(aliases), dtype, shape, stride, off, nbytes, rg, persistent)


def read_manifest(buf: memoryview) -> tuple[list[TensorDescriptor], int]:
    """Validate the header and manifest of a store; returns descriptors and the data offset.

    The segment may be longer than the header says (page rounding); a
    declared range past its end is an error.
    """
    n = len(buf)
    if n < HEADER.size:
        raise RuntimeError("SharedTensorStore header bounds exceed the SHM segment")
    magic, version, mlen, data_offset, data_size = HEADER.unpack_from(buf, 0)
    if magic != MAGIC:
        raise RuntimeError(f"SharedTensorStore magic mismatch: expected {MAGIC!r}, got {magic!r}")
    if version != VERSION:
        raise RuntimeError(f"SharedTensorStore version mismatch: expected {VERSION}, got {version}")
    m_end = HEADER.size + mlen
    if mlen == 0 or m_end > n or data_offset < m_end or data_offset % DATA_ALIGNMENT or data_offset + data_size > n:
        raise RuntimeError("SharedTensorStore header bounds are invalid for the SHM segment")
    try:
        manifest = json.loads(bytes(buf[HEADER.size:m_end]).decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as err:
        raise RuntimeError("SharedTensorStore manifest is not valid UTF-8 JSON") from err
    if not isinstance(manifest, dict) or set(manifest) != {"tensors"} or not isinstance(manifest["tensors"], list):
        raise RuntimeError("SharedTensorStore manifest must contain a tensor descriptor list")
    seen: set[str] = set()
    descs = [_parse_descriptor(v, data_size, seen) for v in manifest["tensors"]]
    ranges = sorted((d.payload_offset, d.payload_offset + d.byte_length) for d in descs if d.byte_length)
    for a, b in pairwise(ranges):
        if b[0] < a[1]:
            raise RuntimeError("SharedTensorStore payload bounds overlap between descriptors")
    return descs, data_offset


class SharedTensorStore:
    """Resident parameters and buffers shared between serving processes (shm/tensor_store.py:415-620).

    A creator publishes one store per namespace; followers attach, validate
    the manifest, and copy the tensors into their own model on their own
    device. Materialized tensors never alias the segment, so closing the
    store leaves them valid.
    """

    def __init__(self, segment: SharedSegment, descriptors: list[TensorDescriptor], data_offset: int) -> None:
        self._segment: SharedSegment | None = segment
        self.descriptors = list(descriptors)
        self.data_offset = data_offset

    @classmethod
    def create_from_model(cls, namespace: str, model: nn.Module, *,
                          parameter_names: Iterable[str]) -> "SharedTensorStore":
        descs, sources, manifest, data_offset, data_size = plan_store(model, parameter_names)
        seg = SharedSegment(store_segment_name(namespace), data_offset + data_size, create=True,
                            initializer=lambda buf: write_store(buf, descs, sources, manifest, data_offset, data_size))
        return cls(seg, descs, data_offset)

    @classmethod
    def attach(cls, namespace: str) -> "SharedTensorStore":
        seg = SharedSegment(store_segment_name(namespace))
        try:
            view = seg.buf[:]
            try:
                descs, data_offset = read_manifest(view)
            finally:
                view.release()
        except BaseException:
            seg.close()
            raise
        return cls(seg, descs, data_offset)

    @property
    def closed(self) -> bool:
        return self._segment is None

    def _validate_target(self, model: nn.Module) -> None:
        params = dict(model.named_parameters(recurse=True, remove_duplicate=False))
        buffers = dict(model.named_buffers(recurse=True, remove_duplicate=False))
        for d in self.descriptors:
            table, other = (params, buffers) if d.kind == "parameter" else (buffers, params)
            for a in d.aliases:
                t = table.get(a)
                if t is None:
                    raise ValueError(f"SharedTensorStore target {d.kind} {a!r} is "
                                     f"{'wrong kind' if a in other else 'missing'}")
                if tuple(t.shape) != d.shape:
                    raise ValueError(f"SharedTensorStore target {a!r} shape mismatch: expected {d.shape}, "
                                     f"got {tuple(t.shape)}")
                # a meta placeholder takes the stored dtype; a concrete target must already have it
                if not t.is_meta and t.dtype != d.dtype:
                    raise ValueError(f"SharedTensorStore target {a!r} dtype mismatch: expected {d.dtype}, "
                                     f"got {t.dtype}")

    def materialize_into(self, model: nn.Module, *, device: torch.device | str, chunk_bytes: int | None = None) -> None:
        """Validate every target, copy every payload to ``device``, then rebind names.

        Nothing in ``model`` changes until every copy has succeeded. On a GPU
        the copies go through pinned staging, one host-link copy and one
        scatter launch per chunk of ``chunk_bytes`` (default 512 MiB).
        """
        seg = self._segment
        if seg is None:
            raise RuntimeError("SharedTensorStore is closed")
        self._validate_target(model)
        dev = torch.device(device)
        view = seg.buf[:]
        try:
            copies = self._copy_out(view, dev, chunk_bytes)
        finally:
            view.release()  # every tensor over the mapping died with _copy_out's frame
        for d, t in zip(self.descriptors, copies):
            obj = nn.Parameter(t, requires_grad=d.requires_grad) if d.kind == "parameter" else t
            for i, a in enumerate(d.aliases):
                parent, leaf = _owner(model, a)
                setattr(parent, leaf, obj)
                if d.kind == "buffer":
                    if d.persistent[i]:
                        parent._non_persistent_buffers_set.discard(leaf)
                    else:
                        parent._non_persistent_buffers_set.add(leaf)

    def _copy_out(self, view: memoryview, dev: torch.device, chunk_bytes: int | None) -> list[torch.Tensor]:
        """Independent copies of every payload on ``dev``, in descriptor order."""
        srcs = [_payload_view(view, self.data_offset, d) for d in self.descriptors if d.byte_length]
        if dev.type == "cuda" and srcs:
            from .scatter import DEFAULT_CHUNK_BYTES, upload_tensors

            placed = iter(upload_tensors(srcs, dev, chunk_bytes=chunk_bytes or DEFAULT_CHUNK_BYTES))
        else:
            placed = iter([t.to(device=dev, copy=True) for t in srcs])
        return [next(placed) if d.byte_length else torch.empty_strided(d.shape, d.stride, dtype=d.dtype, device=dev)
                for d in self.descriptors]

    def close(self) -> None:
        """Unmap (the creator also removes the segment name). Idempotent."""
        seg, self._segment = self._segment, None
        self.descriptors = []
        if seg is not None:
            seg.close()
