"""Stream packed host chunks through a device ring and scatter them into tensors.

This is the batched unpack of the streaming engine and its use for placing
tensors that stay resident on the GPU. The reference moves such tensors to
the device one ``.to()`` / ``copy_`` at a time (tensor_processors.py:685-742;
loaders.py:592-617, 792-797); here they are packed into large pinned chunks,
each chunk crosses the host link in one copy, and one scatter launch per chunk
places its bytes into every destination tensor.

Ordering uses :class:`~flextensor_amd.transfer.HipTransferRuntime`: chunk *i*
is copied on the transfer stream into ring slot ``i % n_slots`` once the
scatter of chunk ``i - n_slots`` released that slot, and its scatter runs on
the caller's stream after the copy's ready event.

Chunks are either packed up front into pinned memory of their own (the
steady state of streaming, :func:`fill_chunks`) or staged: packed on the fly
into a small ring of pinned staging buffers, buffer ``i % n_host`` being
refilled once the copy of chunk ``i - n_host`` out of it has finished, so the
host packing of one chunk overlaps the link transfer of the previous one and
pinned memory stays at ``n_host`` chunks whatever the total.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence
from dataclasses import dataclass, field

import torch

from . import _native as nat
from .hip import HostArena, current_stream
from .layout import DEFAULT_ALIGNMENT, contiguous_strides, is_dense_layout, raw_storage_bytes
from .transfer import HipTransferRuntime

DEFAULT_CHUNK_BYTES = 512 << 20


class ScatterPlan:
    """A device-resident scatter descriptor table (``ftx_scatter_plan``)."""

    def __init__(self, descs: Sequence[tuple[int, int, int]], tile_bytes: int = 0) -> None:
        arr = nat.make_desc_array(descs)
        self._handle = ctypes.c_void_p()
        nat.call("ftx_scatter_plan_create", arr, len(descs), tile_bytes, ctypes.byref(self._handle))
        n_desc, n_tiles, total = ctypes.c_int(0), ctypes.c_int64(0), ctypes.c_uint64(0)
        nat.call("ftx_scatter_plan_info", self._handle, ctypes.byref(n_desc), ctypes.byref(n_tiles),
                 ctypes.byref(total))
        self.n_desc = n_desc.value
        self.n_tiles = n_tiles.value
        self.total_bytes = total.value

    def run(self, chunk: torch.Tensor, stream=None) -> None:
        if chunk.device.type != "cuda":
            raise ValueError("scatter source chunk must be on the device")
        s = stream if stream is not None else current_stream(chunk.device)
        nat.call("ftx_scatter_run", self._handle, chunk.data_ptr(), s.handle)

    def close(self) -> None:
        if self._handle and self._handle.value:
            nat.call("ftx_scatter_plan_destroy", self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self) -> None:
        h = getattr(self, "_handle", None)
        if h is None or not h.value:
            return
        try:
            if nat.live():
                nat.lib().ftx_scatter_plan_destroy(h)
            self._handle = ctypes.c_void_p()
        except (TypeError, AttributeError):
            pass  # interpreter shutdown: module globals are already gone; the process frees the plan


@dataclass
class Piece:
    """``nbytes`` of tensor ``index`` starting at byte ``tensor_off`` live at ``chunk_off``."""

    index: int
    tensor_off: int
    chunk_off: int
    nbytes: int


@dataclass
class Chunk:
    nbytes: int
    pieces: list[Piece] = field(default_factory=list)
    host: torch.Tensor | None = None


def plan_chunks(sizes: Sequence[int], chunk_bytes: int = DEFAULT_CHUNK_BYTES,
                alignment: int = DEFAULT_ALIGNMENT) -> list[Chunk]:
    """Pack tensors in order into chunks of at most ``chunk_bytes``.

    Each piece starts at an ``alignment`` boundary; a tensor that does not fit
    in the space left is split at the chunk boundary and continues at offset 0
    of the next chunk.
    """
    if chunk_bytes <= 0 or chunk_bytes % alignment:
        raise ValueError("chunk_bytes must be a positive multiple of the alignment")
    chunks = [Chunk(0)]
    for i, n in enumerate(sizes):
        done = 0
        while done < n or (n == 0 and done == 0):
            cur = chunks[-1]
            start = -(-cur.nbytes // alignment) * alignment
            if start >= chunk_bytes:
                chunks.append(Chunk(0))
                continue
            take = min(n - done, chunk_bytes - start)
            cur.pieces.append(Piece(i, done, start, take))
            cur.nbytes = start + take
            done += take
            if n == 0:
                break
    if chunks and chunks[-1].nbytes == 0 and not chunks[-1].pieces:
        chunks.pop()
    return chunks


def _source_bytes(t: torch.Tensor) -> torch.Tensor:
    """Raw storage bytes of a dense tensor; a C-contiguous copy's bytes otherwise."""
    if t.numel() == 0:
        return torch.empty(0, dtype=torch.uint8)
    if is_dense_layout(t):
        return raw_storage_bytes(t.detach())
    return t.detach().contiguous().view(-1).view(torch.uint8)


def pack_chunk(host: torch.Tensor, ch: Chunk, tensors: Sequence[torch.Tensor]) -> None:
    """Copy every piece of ``ch`` from ``tensors`` into the host bytes ``host``."""
    if host.numel() < ch.nbytes:
        raise ValueError(f"staging buffer of {host.numel()} bytes cannot hold a {ch.nbytes}-byte chunk")
    for p in ch.pieces:
        if p.nbytes:
            src = _source_bytes(tensors[p.index])
            host[p.chunk_off: p.chunk_off + p.nbytes].copy_(src[p.tensor_off: p.tensor_off + p.nbytes])


def fill_chunks(chunks: Sequence[Chunk], tensors: Sequence[torch.Tensor]) -> None:
    """Allocate one pinned arena per chunk and copy every piece into it."""
    for ch in chunks:
        ch.host = HostArena(max(ch.nbytes, 1)).tensor
        pack_chunk(ch.host, ch, tensors)


def destination_like(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Uninitialised device tensor with ``t``'s layout (dense) or C-contiguous (gapped)."""
    stride = tuple(t.stride()) if is_dense_layout(t) else contiguous_strides(t.shape)
    return torch.empty_strided(tuple(t.shape), stride, dtype=t.dtype, device=device)


def _dst_base(t: torch.Tensor) -> int:
    lowest = t.storage_offset() + sum((k - 1) * s for k, s in zip(t.shape, t.stride()) if s < 0)
    return t.untyped_storage().data_ptr() + lowest * t.element_size()


class ChunkedUploader:
    """Uploads packed chunks into destination tensors through an ``n_slots`` ring."""

    def __init__(self, chunks: Sequence[Chunk], destinations: Sequence[torch.Tensor], device: torch.device,
                 n_slots: int = 2, copy_mode: int = nat.COPY_AUTO, runtime: HipTransferRuntime | None = None,
                 sources: Sequence[torch.Tensor] | None = None, n_host: int = 2) -> None:
        """``sources`` given: chunks without host bytes are staged through ``n_host`` pinned buffers."""
        if n_slots < 1 or n_host < 1:
            raise ValueError("n_slots and n_host must be >= 1")
        self.device = torch.device(device)
        self.chunks = list(chunks)
        self.copy_mode = copy_mode
        self.sources = sources
        staged = [c for c in self.chunks if c.host is None]
        if staged and sources is None:
            raise ValueError("chunks without host bytes need the source tensors to stage from")
        stage_bytes = max((c.nbytes for c in staged), default=0)
        self.staging = [HostArena(max(stage_bytes, 1)).tensor for _ in range(min(n_host, len(staged)))]
        self._staging_free: list = [None] * len(self.staging)  # copy-done event of each staging buffer
        slot_bytes = max((c.nbytes for c in self.chunks), default=1)
        self.n_slots = min(n_slots, max(1, len(self.chunks)))
        self.slots = [torch.empty(max(slot_bytes, 1), dtype=torch.uint8, device=self.device)
                      for _ in range(self.n_slots)]
        self.plans = []
        for ch in self.chunks:
            descs = []
            for p in ch.pieces:
                if p.nbytes:
                    dst = destinations[p.index]
                    if dst.device != self.device:
                        raise ValueError("destination tensors must live on the uploader's device")
                    descs.append((p.chunk_off, _dst_base(dst) + p.tensor_off, p.nbytes))
            self.plans.append(ScatterPlan(descs))
        self.runtime = runtime if runtime is not None else HipTransferRuntime(self.device)
        self.payload_bytes = sum(p.nbytes for ch in self.chunks for p in ch.pieces)

    def upload(self, timing: list | None = None) -> None:
        """Stream every chunk and scatter it; ordered on the caller's current stream.

        With ``timing`` (a list), four timing events per chunk are appended as
        ``(copy_start, copy_end, scatter_start, scatter_end)``: the copy pair
        on the transfer stream around the copy, the scatter pair on the
        caller's stream around the scatter launch.
        """
        from .hip import HipEvent

        rt = self.runtime
        rt.begin()
        n_staged = 0
        for i, ch in enumerate(self.chunks):
            slot = i % self.n_slots
            dst = self.slots[slot]
            ev = [HipEvent(timing=True) for _ in range(4)] if timing is not None else None
            host, stage = ch.host, None
            if host is None:
                stage = n_staged % len(self.staging)
                n_staged += 1
                if self._staging_free[stage] is not None:
                    self._staging_free[stage].synchronize()  # the copy out of this buffer has finished
                host = self.staging[stage]
                pack_chunk(host, ch, self.sources)

            def copy(ch: Chunk = ch, dst: torch.Tensor = dst, ev=ev, host: torch.Tensor = host, stage=stage) -> None:
                s = rt.backend.current_stream()
                if ev:
                    s.record_event(ev[0])
                nat.copy_h2d(dst.data_ptr(), host.data_ptr(), ch.nbytes, self.copy_mode, s.handle)
                if ev:
                    s.record_event(ev[1])
                if stage is not None:
                    self._staging_free[stage] = s.record_event(HipEvent())

            ticket = rt.submit(slot, copy, trace_label=f"chunk={i}")
            rt.wait_ready(ticket)
            if ev:
                rt.backend.current_stream().record_event(ev[2])
            self.plans[i].run(dst)
            if ev:
                rt.backend.current_stream().record_event(ev[3])
                timing.append(tuple(ev))
            rt.finish_use(slot)
        rt.join()

    def close(self) -> None:
        for p in self.plans:
            p.close()
        self.plans = []
        self.slots = []
        self.runtime.close()
        self.staging, self._staging_free, self.sources = [], [], None


def upload_tensors(tensors: Sequence[torch.Tensor], device: torch.device, chunk_bytes: int = DEFAULT_CHUNK_BYTES,
                   n_slots: int = 2, staged: bool = True, n_host: int = 2) -> list[torch.Tensor]:
    """Device copies of host ``tensors`` placed by stream-and-scatter (layouts preserved).

    ``staged`` packs chunk by chunk through ``n_host`` pinned staging buffers
    (pinned memory bounded by ``n_host * chunk_bytes``); otherwise every chunk
    is packed into pinned memory of its own before the first copy.
    """
    device = torch.device(device)
    dests = [destination_like(t, device) for t in tensors]
    chunks = plan_chunks([t.numel() * t.element_size() for t in tensors], chunk_bytes)
    if not staged:
        fill_chunks(chunks, tensors)
    up = ChunkedUploader(chunks, dests, device, n_slots=n_slots, sources=tensors, n_host=n_host)
    try:
        up.upload()
        current_stream(device).synchronize()
    finally:
        up.close()
    return dests
