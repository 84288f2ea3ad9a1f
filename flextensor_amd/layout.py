"""Byte layout of packed label blocks (rows a1/a2 of the hot path).

* :func:`compute_packed_byte_layout` - 128-byte aligned packing offsets
  (utils.py:19-23, 114-127).
* :func:`is_dense_layout` - whether a tensor's elements occupy one gap-free
  span (utils.py:451-476).
* :func:`view_from_block` - a typed, strided view into a ``uint8`` block at a
  byte offset (allocation_block.py:188-207).
* :class:`TensorSlot` - where one tensor lives inside a packed block: byte
  offset, byte count, dtype, shape and the strides the block keeps. Dense
  tensors keep their own strides (C-, Fortran- or any permutation-contiguous);
  tensors with gaps are packed C-contiguous (allocation_block.py:167-177).
"""

from __future__ import annotations

import math
from collections.abc import Iterable, Sequence
from dataclasses import dataclass

import torch

DEFAULT_ALIGNMENT = 128


def _check_alignment(alignment: object) -> int:
    if type(alignment) is not int or alignment <= 0:
        raise ValueError(f"memory_alignment must be a positive integer, got {alignment!r}")
    return alignment


def compute_packed_byte_layout(sizes: Iterable[int], alignment: int = DEFAULT_ALIGNMENT) -> tuple[list[int], int]:
    """Offsets of ``sizes`` packed back to back, each start rounded up to ``alignment``.

    Returns ``(offsets, total)`` where ``total`` is the block size, itself a
    multiple of ``alignment``.
    """
    a = _check_alignment(alignment)
    offsets: list[int] = []
    end = 0
    for n in sizes:
        offsets.append(end)
        end = -(-(end + int(n)) // a) * a
    return offsets, end


def is_dense_layout(t: torch.Tensor) -> bool:
    """True when the ``numel`` elements fill exactly one contiguous span."""
    if t.numel() <= 1 or t.is_contiguous():
        return True
    span = 1 + sum((n - 1) * abs(s) for n, s in zip(t.shape, t.stride()))
    return span == t.numel()


def is_packed_layout(shape: Sequence[int], stride: Sequence[int]) -> bool:
    """Whether a shape/stride pair with non-negative strides covers one gap-free,
    non-overlapping span: taking the dimensions longer than 1 in increasing
    stride order, each stride equals the element count of the dimensions before
    it (utils.py:86-98). Empty shapes qualify."""
    if any(int(n) == 0 for n in shape):
        return True
    span = 1
    for n, s in sorted(((int(n), int(s)) for n, s in zip(shape, stride) if int(n) > 1), key=lambda d: d[1]):
        if s != span:
            return False
        span *= n
    return True


def contiguous_strides(shape: Sequence[int]) -> tuple[int, ...]:
    strides = []
    acc = 1
    for n in reversed(tuple(shape)):
        strides.append(acc)
        acc *= max(int(n), 1)
    return tuple(reversed(strides))


def view_from_block(
    block: torch.Tensor,
    dtype: torch.dtype,
    shape: Sequence[int],
    offset_bytes: int = 0,
    stride: Sequence[int] | None = None,
) -> torch.Tensor:
    """A ``dtype`` view of ``block``'s storage starting ``offset_bytes`` in."""
    itemsize = torch.empty(0, dtype=dtype).element_size()
    if offset_bytes % itemsize != 0:
        raise ValueError(f"offset_bytes ({offset_bytes}) must be a multiple of dtype element size {itemsize}")
    out = torch.empty(0, dtype=dtype, device=block.device)
    base = block.storage_offset() * block.element_size() + offset_bytes
    out.set_(block.untyped_storage(), base // itemsize, tuple(shape),
             tuple(stride) if stride is not None else contiguous_strides(shape))
    return out


def raw_storage_bytes(t: torch.Tensor) -> torch.Tensor:
    """The bytes a dense tensor occupies, in memory order, as a ``uint8`` view."""
    if not is_dense_layout(t):
        raise ValueError("raw_storage_bytes needs a dense tensor")
    n = t.numel() * t.element_size()
    lowest = t.storage_offset() + sum((k - 1) * s for k, s in zip(t.shape, t.stride()) if s < 0)
    raw = torch.empty(0, dtype=torch.uint8, device=t.device)
    raw.set_(t.untyped_storage(), lowest * t.element_size(), (n,))
    return raw


def storage_byte_span(t: torch.Tensor) -> tuple[int, int]:
    """``[lo, hi)``: the bytes of its storage that ``t`` can touch (any strides, including negative)."""
    es = t.element_size()
    lowest = t.storage_offset() + sum((k - 1) * s for k, s in zip(t.shape, t.stride()) if s < 0)
    extent = 1 + sum((k - 1) * abs(s) for k, s in zip(t.shape, t.stride()))
    return lowest * es, (lowest + extent) * es


def overlapping_views(managed: Iterable[torch.Tensor], others: Iterable[torch.Tensor] = ()) -> list[list[int]]:
    """Groups of distinct tensors (by ``id``) whose byte ranges overlap within one storage, each group
    holding at least one ``managed`` tensor. Disjoint views of one storage are not reported."""
    groups: dict[tuple[str, int], list[tuple[int, int, int, bool]]] = {}
    seen: set[int] = set()
    for flag, ts in ((True, managed), (False, others)):
        for t in ts:
            if id(t) in seen or t.is_meta or t.layout != torch.strided or t.numel() == 0:
                continue
            seen.add(id(t))
            st = t.untyped_storage()
            if st.nbytes() == 0:
                continue
            lo, hi = storage_byte_span(t)
            groups.setdefault((str(t.device), st.data_ptr()), []).append((lo, hi, id(t), flag))
    out: list[list[int]] = []

    def flush(cluster: list[tuple[int, int, int, bool]]) -> None:
        if len(cluster) > 1 and any(c[3] for c in cluster):
            out.append(sorted(c[2] for c in cluster))

    for spans in groups.values():
        spans.sort()
        cluster, end = [spans[0]], spans[0][1]
        for span in spans[1:]:
            if span[0] < end:  # starts inside the cluster's reach: overlaps one of its members
                cluster.append(span)
                end = max(end, span[1])
            else:
                flush(cluster)
                cluster, end = [span], span[1]
        flush(cluster)
    return out


@dataclass(frozen=True)
class TensorSlot:
    """Placement of one tensor inside a packed block."""

    offset: int
    nbytes: int
    dtype: torch.dtype
    shape: tuple[int, ...]
    stride: tuple[int, ...]

    @staticmethod
    def for_tensor(t: torch.Tensor, offset: int) -> "TensorSlot":
        keep = is_dense_layout(t)
        stride = tuple(t.stride()) if keep else contiguous_strides(t.shape)
        return TensorSlot(offset, t.numel() * t.element_size(), t.dtype, tuple(t.shape), stride)

    def view(self, block: torch.Tensor) -> torch.Tensor:
        return view_from_block(block, self.dtype, self.shape, self.offset, self.stride)


def plan_block(tensors: Sequence[torch.Tensor], alignment: int = DEFAULT_ALIGNMENT) -> tuple[list[TensorSlot], int]:
    """Slots for ``tensors`` packed into one block, and the block size."""
    sizes = [t.numel() * t.element_size() for t in tensors]
    offsets, total = compute_packed_byte_layout(sizes, alignment)
    return [TensorSlot.for_tensor(t, off) for t, off in zip(tensors, offsets)], total


def pack_into(block: torch.Tensor, slots: Sequence[TensorSlot], tensors: Sequence[torch.Tensor]) -> list[torch.Tensor]:
    """Copy every tensor into its slot of a host block; returns the typed views.

    A dense tensor is copied as raw storage bytes, so the block holds the
    bytes in the tensor's own memory order; a tensor with gaps is copied
    element-wise into a C-contiguous slot. The alignment gaps between slots
    and after the last are zeroed, so a block's bytes depend only on its
    tensors.
    """
    pos = 0
    flat = block.view(torch.uint8).reshape(-1)
    for slot in sorted(slots, key=lambda x: x.offset):
        if slot.offset > pos:
            flat[pos:slot.offset].zero_()
        pos = max(pos, slot.offset + slot.nbytes)
    if flat.numel() > pos:
        flat[pos:].zero_()
    views = []
    for slot, t in zip(slots, tensors):
        view = slot.view(block)
        if t.numel():
            if is_dense_layout(t) and tuple(t.stride()) == slot.stride:
                dst = view_from_block(block, torch.uint8, (slot.nbytes,), slot.offset)
                dst.copy_(raw_storage_bytes(t.detach()))
            else:
                view.copy_(t.detach())
        views.append(view)
    return views


def total_bytes(tensors: Iterable[torch.Tensor]) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def numel(shape: Sequence[int]) -> int:
    return math.prod(int(x) for x in shape)
