"""Oracle: packed byte layout and dense-layout rules, restated on plain tuples.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations


def packed_layout(sizes, alignment=128):
    """Offsets and total of aligned back-to-back packing (utils.py:114-127)."""
    if type(alignment) is not int or alignment <= 0:
        raise ValueError(f"memory_alignment must be a positive integer, got {alignment!r}")
    offsets, cursor = [], 0
    for size in sizes:
        offsets.append(cursor)
        cursor += size
        cursor = ((cursor + alignment - 1) // alignment) * alignment
    return offsets, cursor


def raw_layout(sizes):
    """Back-to-back offsets with no alignment (loaders.py:1007-1028)."""
    offsets, cursor = [], 0
    for size in sizes:
        offsets.append(cursor)
        cursor += size
    return offsets, cursor


def is_dense(shape, stride):
    """Elements fill one gap-free span (utils.py:451-476): C-contiguous, or
    max offset + 1 == numel."""
    numel = 1
    for s in shape:
        numel *= s
    if numel <= 1:
        return True
    c_stride, expect = [], 1
    for s in reversed(shape):
        c_stride.append(expect)
        expect *= s
    c_stride.reverse()
    if all(st == cs for st, cs, s in zip(stride, c_stride, shape) if s != 1):
        return True
    return sum((s - 1) * abs(st) for s, st in zip(shape, stride)) + 1 == numel


def packed_strides(shape, stride):
    """Strides a tensor keeps inside a block: its own when dense, C-contiguous
    otherwise (allocation_block.py:167-177)."""
    if is_dense(shape, stride):
        return tuple(stride)
    out, acc = [], 1
    for s in reversed(shape):
        out.append(acc)
        acc *= max(s, 1)
    return tuple(reversed(out))
