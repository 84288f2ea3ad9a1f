"""Exponent-coded blocks: a streamed block carried over the link in about 0.70 of its bytes, a resident
one kept in HBM in as few.

No reference counterpart: the reference copies each label's packed block as raw bytes
(allocation_block.py:104-106). With ``OffloadConfig.encode_streamed_blocks`` the block controller keeps,
beside each streamed label's pinned raw block, an encoded copy in a pinned, device-mapped arena, and
its host-to-device transfer becomes one decode launch (``ftx_expcode_decode_h2d``): a zero-copy kernel
reads the encoded bytes over the link and writes the raw bytes into the ring slot, bit for bit.

Two formats. Version 1 (``FTXE`` v1, ``ftx_expcode_encode``) codes each bf16 word's exponent in 4 bits
for the block's 15 most frequent exponents, with the rest as escapes: 0.752 of the bytes. The dense
version 2 (``ftx_expcode_encode_dense``) codes the 7 most frequent in 3 bits and the next 15 in a 4-bit
secondary code per escape: 0.697. Its decoders rank escapes across the wave before reading their
codes; the controllers use it for every block, and ``ftx_expcode_decode_h2d`` reads a block's version
from its header. The encoders are the library's host routines.

With ``OffloadConfig.encode_resident_blocks`` resident units are kept encoded in device memory instead
(:class:`DeviceEncodedBlock`): more units fit the GPU budget, fewer stream, and each such unit is
decoded from HBM (``ftx_expcode_decode_dense_d2d``) into one shared slot on the compute stream as it
runs.
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


def encoded_size(raw: torch.Tensor, dense: bool = False) -> int:
    """Bytes of the encoded block for ``raw`` (a contiguous CPU tensor, read as bytes); ``dense``: of the
    dense format (version 2) that units kept in device memory use."""
    ptr, n = _raw_ptr(raw)
    out = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode_dense" if dense else "ftx_expcode_encode", ptr, n, None, 0, ctypes.byref(out))
    return int(out.value)


class EncodedBlock:
    """One raw block encoded into a pinned, device-mapped host arena of ``arena.nbytes`` bytes.

    The arena may hold more than the encoded ``nbytes``: :meth:`reencode` rewrites the block in place
    (same arena, so decode launches captured in a graph stay valid, and they read the new header when
    they run) as long as the new encoding fits."""

    __slots__ = ("arena", "nbytes", "raw_bytes", "dense")

    def __init__(self, arena: HostArena, nbytes: int, raw_bytes: int, dense: bool = False) -> None:
        self.arena = arena
        self.nbytes = int(nbytes)
        self.raw_bytes = int(raw_bytes)
        self.dense = bool(dense)  # the dense format (version 2); the decode reads the version from the header

    def reencode(self, raw: torch.Tensor) -> None:
        """Encode ``raw`` (the same raw size) into this block's arena. No decode of this block may be in
        flight. Raises ValueError when the new encoding does not fit the arena."""
        ptr, n = _raw_ptr(raw)
        if n != self.raw_bytes:
            raise ValueError(f"raw block of {n} bytes, but this block encodes {self.raw_bytes}")
        size = encoded_size(raw, self.dense)
        if size > self.arena.nbytes:
            raise ValueError(f"the new encoding needs {size} bytes, more than the {self.arena.nbytes} of its arena")
        out = ctypes.c_size_t(0)
        nat.call("ftx_expcode_encode_dense" if self.dense else "ftx_expcode_encode", ptr, n, self.arena.ptr,
                 self.arena.nbytes, ctypes.byref(out))
        self.nbytes = int(out.value)

    @property
    def ratio(self) -> float:
        return self.nbytes / self.raw_bytes if self.raw_bytes else 1.0

    @property
    def tensor(self) -> torch.Tensor:
        """The encoded bytes (a CPU view of the arena)."""
        return self.arena.tensor[: self.nbytes]


def encode(raw: torch.Tensor, size: int | None = None, capacity: int = 0, dense: bool = False) -> EncodedBlock:
    """Encode ``raw`` into a new arena of at least ``capacity`` bytes (``size``: the encoded size, if
    already known), in the dense format (version 2) when ``dense``."""
    ptr, n = _raw_ptr(raw)
    size = encoded_size(raw, dense) if size is None else int(size)
    arena = HostArena(max(size, int(capacity), 1))
    out = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode_dense" if dense else "ftx_expcode_encode", ptr, n, arena.ptr, arena.nbytes,
             ctypes.byref(out))
    if out.value != size:
        raise RuntimeError(f"encoded size {out.value} differs from the {size} bytes planned")
    return EncodedBlock(arena, size, n, dense)


def encode_if_smaller(raw: torch.Tensor, max_ratio: float = DEFAULT_MAX_RATIO,
                      dense: bool = False) -> EncodedBlock | None:
    """The encoded block, or None when it would not be below ``max_ratio`` of the raw size. Its arena
    holds the raw size, so any later contents that encode no larger than raw re-encode in place."""
    _, n = _raw_ptr(raw)
    if n == 0:
        return None
    size = encoded_size(raw, dense)
    if size > max_ratio * n:
        return None
    return encode(raw, size, capacity=n, dense=dense)


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


def packed_encoded_size(tensors: list[torch.Tensor], alignment: int, scratch: torch.Tensor | None = None,
                        dense: bool = False) -> tuple[int, int]:
    """(encoded bytes, raw bytes) of the block that packs ``tensors`` (CPU) at ``alignment``, as a block
    controller packs them: gaps zeroed, so the size is exact. ``scratch`` (uint8, CPU), when large enough,
    holds the packed bytes instead of a new buffer; ``dense`` sizes the dense format (version 2)."""
    from .layout import pack_into, plan_block

    slots, total = plan_block(tensors, alignment)
    if total == 0:
        return 0, 0
    buf = scratch[:total] if scratch is not None and scratch.numel() >= total else torch.empty(total,
                                                                                                 dtype=torch.uint8)
    pack_into(buf, slots, tensors)
    return encoded_size(buf, dense), total


class DeviceEncodedBlock:
    """An encoded block kept in device memory: ``dev`` (uint8, ``capacity`` bytes) holds ``nbytes`` of
    encoded bytes for a raw block of ``raw_bytes``, in the dense format (version 2) when ``dense``, else
    in version 1. Serves units kept resident in HBM in encoded form: :meth:`decode` rebuilds the raw block
    on the device before the unit runs.

    :meth:`reencode` rewrites the block in place (same device buffer, so decodes captured in a graph stay
    valid and read the new header when they run) as long as the new encoding fits ``capacity``."""

    __slots__ = ("dev", "nbytes", "raw_bytes", "dense")

    def __init__(self, dev: torch.Tensor, nbytes: int, raw_bytes: int, dense: bool = False) -> None:
        self.dev = dev
        self.nbytes = int(nbytes)
        self.raw_bytes = int(raw_bytes)
        self.dense = bool(dense)

    @staticmethod
    def _encode_host(raw: torch.Tensor, dense: bool) -> torch.Tensor:
        ptr, n = _raw_ptr(raw)
        size = encoded_size(raw, dense)
        host = torch.empty(max(size, 1), dtype=torch.uint8)
        out = ctypes.c_size_t(0)
        nat.call("ftx_expcode_encode_dense" if dense else "ftx_expcode_encode", ptr, n, host.data_ptr(),
                 host.numel(), ctypes.byref(out))
        return host[: out.value]

    @classmethod
    def from_raw(cls, raw: torch.Tensor, capacity: int, device: torch.device,
                 dense: bool = False) -> "DeviceEncodedBlock":
        """Encode ``raw`` (contiguous CPU) into a new device buffer of ``capacity`` bytes."""
        host = cls._encode_host(raw, dense)
        if host.numel() > capacity:
            raise ValueError(f"the encoding needs {host.numel()} bytes, more than its capacity of {capacity}")
        dev = torch.empty(max(int(capacity), 16), dtype=torch.uint8, device=device)
        dev[: host.numel()].copy_(host)
        return cls(dev, host.numel(), raw.numel() * raw.element_size(), dense)

    @property
    def capacity(self) -> int:
        return self.dev.numel()

    @property
    def ratio(self) -> float:
        return self.nbytes / self.raw_bytes if self.raw_bytes else 1.0

    def reencode(self, raw: torch.Tensor) -> None:
        """Encode ``raw`` (the same raw size) into this block's device buffer; the copy completes before
        this returns. No decode of this block may be in flight. Raises ValueError (and leaves the block
        unchanged) when the new encoding does not fit the capacity."""
        n = raw.numel() * raw.element_size()
        if n != self.raw_bytes:
            raise ValueError(f"raw block of {n} bytes, but this block encodes {self.raw_bytes}")
        host = self._encode_host(raw, self.dense)
        if host.numel() > self.capacity:
            raise ValueError(f"the new encoding needs {host.numel()} bytes, more than the {self.capacity} "
                             "reserved on the device")
        self.dev[: host.numel()].copy_(host)
        torch.cuda.synchronize(self.dev.device)
        self.nbytes = host.numel()

    def decode(self, dst: torch.Tensor, stream: HipStream | None = None) -> None:
        """Stream-ordered decode into the first ``raw_bytes`` bytes of ``dst`` (the library's default grid)."""
        decode_d2d(dst, self.dev, self.raw_bytes, stream, dense=self.dense)


def decode_d2d(dst: torch.Tensor, encoded: torch.Tensor, raw_bytes: int, stream: HipStream | None = None,
               grid: int = 0, dense: bool = False) -> None:
    """Stream-ordered decode of an encoded block held in device memory (``encoded``, a uint8 device tensor)
    into the first ``raw_bytes`` bytes of ``dst``; ``grid`` 0 runs eight workgroups per CU for version 1 and
    sixteen for the dense format (``dense``, version 2)."""
    if dst.device.type != "cuda" or encoded.device.type != "cuda":
        raise ValueError("decode_d2d needs device tensors")
    if raw_bytes > dst.numel() * dst.element_size():
        raise ValueError(f"decoded block of {raw_bytes} bytes does not fit destination of "
                         f"{dst.numel() * dst.element_size()} bytes")
    s = stream if stream is not None else current_stream(dst.device)
    nat.call("ftx_expcode_decode_dense_d2d" if dense else "ftx_expcode_decode_d2d", dst.data_ptr(),
             encoded.data_ptr(), encoded.numel(), raw_bytes, int(grid), s.handle)
