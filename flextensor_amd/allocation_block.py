"""Pinned per-label blocks and their GPU ring slots (rows a2-a5 of the hot path).

An :class:`AllocationBlock` packs one label's tensors byte for byte into a
single page-locked host block at 128-byte aligned offsets, keeps dense
strides (allocation_block.py:124-186), projects typed views at the same byte
offsets into a GPU slot (:81-102) and fills that slot with one stream-ordered
host-to-device copy (:104-106). The copy goes through the C ABI
(``ftx_copy_h2d``), which picks the SDMA engines or the zero-copy kernel per
chunk size. :class:`AllocationManager.create_max_block` sizes a GPU slot to
the largest block of its labels (:260-280).

:class:`HostPinner` replaces the reference's host pinning
(host_pinning.py:374-519): ``"torch"`` mode allocates the block directly in a
pinned arena (no second copy), ``"host_register"`` page-locks an existing
pageable block in place through ``ftx_arena_register``.
"""

from __future__ import annotations

import logging
import threading
from collections.abc import Sequence
from typing import Any

import torch

from . import _native as nat
from .layout import DEFAULT_ALIGNMENT, TensorSlot, _check_alignment, pack_into, plan_block, view_from_block

LOGGER = logging.getLogger(__name__)

PINNED_MEMORY_MODES = ("torch", "host_register")


class HostPinner:
    """Provides page-locked host blocks and keeps a registry of in-place pins."""

    def __init__(self, mode: str = "torch", enabled: bool = True) -> None:
        if mode not in PINNED_MEMORY_MODES:
            raise ValueError(f"pinned_memory_mode must be one of {PINNED_MEMORY_MODES}, got {mode!r}")
        self.mode = mode
        self.enabled = enabled
        # host_register mode: ptr -> (bytes, tensor). The pinner holds the
        # tensor so the memory stays valid while registered; pins end only in
        # release()/release_all() (the reference releases pins at manager
        # shutdown, not with the blocks: host_pinning.py:314-344).
        self._registered: dict[int, tuple[int, torch.Tensor]] = {}
        self._lock = threading.Lock()

    def new_block(self, nbytes: int) -> torch.Tensor:
        """A host ``uint8`` block of ``nbytes``; pinned unless pinning is disabled."""
        n = max(int(nbytes), 1)
        if not self.enabled:
            return torch.empty(n, dtype=torch.uint8)
        if self.mode == "torch":
            from .hip import HostArena

            return HostArena(n).tensor
        block = torch.empty(n, dtype=torch.uint8)
        self.pin_in_place(block)
        return block

    def pin_in_place(self, block: torch.Tensor) -> torch.Tensor:
        """Page-lock the whole storage behind ``block`` once; views of a storage
        already registered register nothing (host_pinning.py:96-122)."""
        storage = block.untyped_storage()
        ptr, nbytes = storage.data_ptr(), storage.nbytes()
        with self._lock:
            if ptr in self._registered:
                return block
            nat.arena_register(ptr, nbytes)
            self._registered[ptr] = (nbytes, block)
        return block

    @staticmethod
    def _should_skip_pin(tensor: torch.Tensor) -> bool:
        """Non-CPU, meta and empty tensors cannot be pinned and already pinned ones
        need not be (host_pinning.py:57-65)."""
        if tensor.device.type != "cpu" or tensor.is_meta or tensor.numel() == 0:
            return True
        return bool(tensor.is_pinned())

    def pin(self, tensor: torch.Tensor) -> torch.Tensor:
        """A pinned tensor with the same contents: ``torch`` mode returns a pinned
        copy, ``host_register`` pins the storage in place and returns ``tensor``.
        Tensors that cannot or need not be pinned come back unchanged, and a
        failure to pin raises (host_pinning.py:28-54)."""
        if not self.enabled or self._should_skip_pin(tensor):
            return tensor
        if self.mode == "host_register":
            return self.pin_in_place(tensor)
        block = self.new_block(tensor.numel() * tensor.element_size())
        out = view_from_block(block, tensor.dtype, tuple(tensor.shape), 0, None)
        out.copy_(tensor)
        return out

    def is_pinned(self, tensor: torch.Tensor) -> bool:
        """``tensor.is_pinned()``, or in ``host_register`` mode whether this pinner
        registered the tensor's storage (registration does not set torch's flag).
        A tensor whose storage yields no pointer reads as not pinned
        (host_pinning.py:67-88)."""
        if tensor.is_pinned():
            return True
        if self.mode != "host_register":
            return False
        try:
            ptr = tensor.untyped_storage().data_ptr()
        except Exception:  # noqa: BLE001 - lazy or fake tensors without a storage pointer
            LOGGER.debug("HostPinner.is_pinned: the tensor's storage has no data pointer; treating it as not pinned")
            return False
        with self._lock:
            return ptr in self._registered

    def release(self, ptr: int) -> None:
        with self._lock:
            if self._registered.pop(ptr, None) is not None:
                nat.arena_unregister(ptr)

    def release_all(self) -> None:
        with self._lock:
            ptrs = list(self._registered)
            self._registered.clear()
        for p in ptrs:
            nat.arena_unregister(p)

    @property
    def pinned_bytes(self) -> int:
        return sum(n for n, _ in self._registered.values())


class AllocationBlock:
    """One label's packed host block (``device="cpu"``) or a GPU ring slot.

    With ``shm_block_name`` the host block is a named POSIX shared-memory
    segment (allocation_block.py:133-158): the creator packs the tensors into
    a new segment and publishes it; with ``load_from_shm`` a follower maps the
    published segment and only builds views (its tensors supply shapes,
    dtypes and strides, not bytes). Such a block is page-locked in place only
    in ``host_register`` pinning mode; otherwise it stays pageable and its
    copies go through the staged copy engine.
    """

    def __init__(
        self,
        manager: Any = None,
        device: str | torch.device = "cpu",
        block_size: int | None = None,
        *,
        host_pinner: HostPinner,
        pinned_memory: bool = True,
        memory_alignment: int = DEFAULT_ALIGNMENT,
        release_tensor_memory: bool = False,
        shm_block_name: str | None = None,
        load_from_shm: bool = False,
    ) -> None:
        if load_from_shm and shm_block_name is None:
            raise ValueError("load_from_shm needs shm_block_name")
        self.manager = manager
        self.device = torch.device(device)
        self.host_pinner = host_pinner
        self.pinned_memory = pinned_memory
        self.shm_block_name = shm_block_name if self.device.type == "cpu" else None
        self.load_from_shm = load_from_shm
        self.shm_segment: Any = None
        self.memory_alignment = _check_alignment(memory_alignment)
        self.release_tensor_memory = release_tensor_memory
        self.tensors: list[torch.Tensor] = []
        self.slots: list[TensorSlot] = []
        self.views: list[torch.Tensor] = []
        self.block: torch.Tensor | None = self._new_block(block_size) if block_size is not None else None

    @property
    def tensor_offsets(self) -> list[int]:
        return [s.offset for s in self.slots]

    @property
    def nbytes(self) -> int:
        return 0 if self.block is None else self.block.numel()

    def _new_block(self, nbytes: int) -> torch.Tensor:
        if int(nbytes) <= 0:  # nothing to hold (create_max_block over uncommitted blocks): no pin, no allocation
            return torch.empty(0, dtype=torch.uint8, device=self.device)
        if self.device.type == "cpu":
            if self.pinned_memory:
                return self.host_pinner.new_block(nbytes)
            return torch.empty(max(int(nbytes), 1), dtype=torch.uint8)
        return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=self.device)

    def _require_block(self) -> torch.Tensor:
        if self.block is None:
            raise RuntimeError("Allocation block is not prepared")
        return self.block

    def add(self, tensor: torch.Tensor) -> None:
        self.tensors.append(tensor)

    @property
    def is_memory_creator(self) -> bool:
        return self.shm_block_name is not None and not self.load_from_shm

    def _shm_block(self, total: int) -> torch.Tensor:
        from .shm import SharedSegment

        size = max(int(total), 1)
        if self.load_from_shm:
            seg = SharedSegment(self.shm_block_name)
            if seg.size < size:
                have = seg.size
                seg.close()
                raise ValueError(f"shared block {self.shm_block_name!r} holds {have} bytes, its tensors need {size}")
        else:
            slots, tensors = self.slots, self.tensors

            def fill(buf: memoryview) -> None:
                pack_into(torch.frombuffer(buf, dtype=torch.uint8), slots, tensors)

            seg = SharedSegment(self.shm_block_name, size, create=True, initializer=fill)
        self.shm_segment = seg
        block = torch.frombuffer(seg.buf, dtype=torch.uint8, count=size)
        if self.pinned_memory and self.host_pinner.enabled and self.host_pinner.mode == "host_register":
            self.host_pinner.pin_in_place(block)
        return block

    def allocate(self) -> list[torch.Tensor]:
        """Pack the added tensors; returns host views that alias the block."""
        self.slots, total = plan_block(self.tensors, self.memory_alignment)
        if self.shm_block_name is not None:
            self.block = self._shm_block(total)
            self.views = [s.view(self.block) for s in self.slots]
        else:
            self.block = self._new_block(total)
            self.views = pack_into(self.block, self.slots, self.tensors)
        if self.release_tensor_memory:
            for t in self.tensors:
                t.data = torch.empty(0, dtype=t.dtype)
        self.tensors.clear()
        return self.views

    def project_views(self, gpu_block: "AllocationBlock") -> tuple[list[torch.Tensor], torch.Tensor]:
        """Typed views into ``gpu_block`` at this block's offsets, and the slot prefix the block fills."""
        block = self._require_block()
        slot = gpu_block._require_block()
        if block.numel() > slot.numel():
            raise ValueError(f"block of {block.numel()} bytes does not fit slot of {slot.numel()} bytes")
        return [s.view(slot) for s in self.slots], slot[: block.numel()]

    def copy_to(self, gpu_view: torch.Tensor, non_blocking: bool = True, stream: Any = None,
                mode: int = nat.COPY_AUTO, policy: nat.CopyPolicy | None = None) -> None:
        """Copy the whole block into ``gpu_view`` on ``stream`` (default: current stream), under the copy
        ``policy`` of the caller (None: the library default)."""
        from .hip import copy_h2d

        block = self._require_block()
        if gpu_view.device.type != "cuda":
            gpu_view.copy_(block)
            return
        copy_h2d(gpu_view, block, mode, stream, policy=policy)
        if not non_blocking:
            (stream if stream is not None else _current(gpu_view.device)).synchronize()

    def release(self) -> None:
        self.block = None
        self.views = []
        self.slots = []
        self.tensors = []
        seg = self.shm_segment
        if seg is not None:
            # The creator removes the name; other processes' mappings stay valid. Closing
            # drops the block's hold on the mapping: tensors that still view it (restored
            # parameters, user references) keep it mapped until the last of them goes.
            # An in-place pin of the mapping ends with the pinner's release_all(), like
            # every other pin (pins are released at manager shutdown, not with blocks).
            # A failed unlink keeps the segment, so release() can be retried.
            seg.close()
        self.shm_segment = None


def _current(device: torch.device):
    from .hip import current_stream

    return current_stream(device)


class AllocationManager:
    """Creates the host blocks of a slot group and the GPU slot that fits them all."""

    def __init__(
        self,
        *,
        host_pinner: HostPinner,
        pinned_memory: bool = True,
        memory_alignment: int = DEFAULT_ALIGNMENT,
        release_tensor_memory: bool = False,
    ) -> None:
        self.blocks: list[AllocationBlock] = []
        self.host_pinner = host_pinner
        self.pinned_memory = pinned_memory
        self.memory_alignment = memory_alignment
        self.release_tensor_memory = release_tensor_memory

    def block(self, device: str | torch.device = "cpu", *, shm_block_name: str | None = None,
              load_from_shm: bool = False) -> AllocationBlock:
        b = AllocationBlock(
            self,
            device=device,
            host_pinner=self.host_pinner,
            pinned_memory=self.pinned_memory,
            memory_alignment=self.memory_alignment,
            release_tensor_memory=self.release_tensor_memory,
            shm_block_name=shm_block_name,
            load_from_shm=load_from_shm,
        )
        self.blocks.append(b)
        return b

    def create_max_block(self, device: str | torch.device = "cuda") -> AllocationBlock:
        largest = max((b.nbytes for b in self.blocks if b.block is not None), default=0)
        return AllocationBlock(self, device=device, block_size=largest, host_pinner=self.host_pinner,
                               pinned_memory=False, memory_alignment=self.memory_alignment)

    def release(self) -> None:
        for b in self.blocks:
            b.release()
        self.blocks = []


def copy_tensors_to_host_block(tensors: Sequence[torch.Tensor], pinner: HostPinner,
                               alignment: int = DEFAULT_ALIGNMENT) -> tuple[torch.Tensor, list[TensorSlot]]:
    """Pack ``tensors`` into one new (pinned) host block; returns the block and slots."""
    slots, total = plan_block(tensors, alignment)
    block = pinner.new_block(total)
    pack_into(block, slots, tensors)
    return block, slots
