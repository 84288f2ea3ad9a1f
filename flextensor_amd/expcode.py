"""Exponent-coded host blocks: a streamed block carried over the link in about 0.75 of its bytes.

No reference counterpart: the reference copies each label's packed block as raw bytes
(allocation_block.py:104-106). With ``OffloadConfig.encode_streamed_blocks`` the block controller keeps,
beside each streamed label's pinned raw block, an encoded copy in a pinned, device-mapped arena, and
its host-to-device transfer becomes one decode launch (``ftx_expcode_decode_h2d``): a zero-copy kernel
reads the encoded bytes over the link and writes the raw bytes into the ring slot, bit for bit. The
format (``FTXE`` v1) codes each bf16 word's exponent in 4 bits for the block's 15 most frequent
exponents, with the rest as escapes; the encoder is the library's host routine
(``ftx_expcode_encode``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat
from .hip import HipStream, HostArena, current_stream

# A block is kept encoded only when this saves at least a tenth of its bytes.
DEFAULT_MAX_RATIO = 0.9


def _raw_ptr(raw: torch.Tensor) -> tuple[int, int]:
    if raw.device.type != "cpu" or not raw.is_contiguous():
        raise ValueError("the raw block must be a contiguous CPU tensor")
    return raw.data_ptr(), raw.numel() * raw.element_size()


def encoded_size(raw: torch.Tensor) -> int:
    """Bytes of the encoded block for ``raw`` (a contiguous CPU tensor, read as bytes)."""
    ptr, n = _raw_ptr(raw)
    out = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode", ptr, n, None, 0, ctypes.byref(out))
    return int(out.value)


class EncodedBlock:
    """One raw block encoded into a pinned, device-mapped host arena of ``arena.nbytes`` bytes.

    The arena may hold more than the encoded ``nbytes``: :meth:`reencode` rewrites the block in place
    (same arena, so decode launches captured in a graph stay valid, and they read the new header when
    they run) as long as the new encoding fits."""

    __slots__ = ("arena", "nbytes", "raw_bytes")

    def __init__(self, arena: HostArena, nbytes: int, raw_bytes: int) -> None:
        self.arena = arena
        self.nbytes = int(nbytes)
        self.raw_bytes = int(raw_bytes)

    def reencode(self, raw: torch.Tensor) -> None:
        """Encode ``raw`` (the same raw size) into this block's arena. No decode of this block may be in
        flight. Raises ValueError when the new encoding does not fit the arena."""
        ptr, n = _raw_ptr(raw)
        if n != self.raw_bytes:
            raise ValueError(f"raw block of {n} bytes, but this block encodes {self.raw_bytes}")
        size = encoded_size(raw)
        if size > self.arena.nbytes:
            raise ValueError(f"the new encoding needs {size} bytes, more than the {self.arena.nbytes} of its arena")
        out = ctypes.c_size_t(0)
        nat.call("ftx_expcode_encode", ptr, n, self.arena.ptr, self.arena.nbytes, ctypes.byref(out))
        self.nbytes = int(out.value)

    @property
    def ratio(self) -> float:
        return self.nbytes / self.raw_bytes if self.raw_bytes else 1.0

    @property
    def tensor(self) -> torch.Tensor:
        """The encoded bytes (a CPU view of the arena)."""
        return self.arena.tensor[: self.nbytes]


def encode(raw: torch.Tensor, size: int | None = None, capacity: int = 0) -> EncodedBlock:
    """Encode ``raw`` into a new arena of at least ``capacity`` bytes (``size``: the encoded size, if
    already known)."""
    ptr, n = _raw_ptr(raw)
    size = encoded_size(raw) if size is None else int(size)
    arena = HostArena(max(size, int(capacity), 1))
    out = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode", ptr, n, arena.ptr, arena.nbytes, ctypes.byref(out))
    if out.value != size:
        raise RuntimeError(f"encoded size {out.value} differs from the {size} bytes planned")
    return EncodedBlock(arena, size, n)


def encode_if_smaller(raw: torch.Tensor, max_ratio: float = DEFAULT_MAX_RATIO) -> EncodedBlock | None:
    """The encoded block, or None when it would not be below ``max_ratio`` of the raw size. Its arena
    holds the raw size, so any later contents that encode no larger than raw re-encode in place."""
    _, n = _raw_ptr(raw)
    if n == 0:
        return None
    size = encoded_size(raw)
    if size > max_ratio * n:
        return None
    return encode(raw, size, capacity=n)


def decode_h2d(dst: torch.Tensor, block: EncodedBlock, stream: HipStream | None = None,
               policy: nat.CopyPolicy | None = None) -> None:
    """Stream-ordered decode of ``block`` into the first ``block.raw_bytes`` bytes of ``dst`` (a device
    tensor); ``policy.kernel_grid`` sets the decode kernel's workgroups (None or 0: the library's 16)."""
    if dst.device.type != "cuda":
        raise ValueError("decode_h2d needs a device destination")
    if block.raw_bytes > dst.numel() * dst.element_size():
        raise ValueError(f"decoded block of {block.raw_bytes} bytes does not fit destination of "
                         f"{dst.numel() * dst.element_size()} bytes")
    s = stream if stream is not None else current_stream(dst.device)
    pol = ctypes.byref(policy) if policy is not None else None
    nat.call("ftx_expcode_decode_h2d", dst.data_ptr(), block.arena.ptr, block.arena.nbytes, pol, s.handle)
