"""Block controllers: own the pinned label blocks and the GPU ring slots.

:class:`AllocationBlockController` follows the reference controller of the
same name (loaders.py:1104-1416): one 128-byte aligned pinned block per
label, one GPU slot per slot group sized to the group's largest block, typed
GPU views at the same byte offsets (the model's parameters alias them), and
``schedule_transfer(label)`` = one host-to-device copy of the label's block
into its slot on the current (transfer) stream.

Each controller carries its own copy engine (``copy_mode``) and copy policy
(``copy_policy``, a :class:`~flextensor_amd._native.CopyPolicy` passed with
every copy; None copies under the library default), so managers that stream
side by side in one process each copy as their own link measurement chose,
as the reference's named managers copy independently
(offload_manager.py:2817-2850).

:class:`RawBlockController` follows ``RawBlockController`` (loaders.py:903-1101):
back-to-back packing without alignment; dense tensors are copied as raw
storage bytes, tensors with gaps as C-contiguous copies.

Failures during construction restore every source tensor that had already
been packed and released (the reference's construction rollback,
loaders.py:1194-1207) before the error propagates.
"""

from __future__ import annotations

import logging
import math
from collections.abc import Mapping, Sequence
from typing import Any

import torch
from torch.multiprocessing.reductions import StorageWeakRef

from . import _native as nat
from .allocation_block import AllocationBlock, AllocationManager, HostPinner
from .layout import contiguous_strides, is_dense_layout, overlapping_views, raw_storage_bytes, view_from_block
from .planner import TensorStatistics

LOGGER = logging.getLogger(__name__)


CLEANUP_NOTE = ("construction cleanup is incomplete; call exception._flextensor_cleanup_controller.shutdown() "
                "to retry it.")


def _cleanup_keeping_error(controller: Any, primary: BaseException) -> None:
    """Undo a failed build; a failing cleanup never replaces ``primary``.

    The controller stays reachable from the primary error as
    ``_flextensor_cleanup_controller`` (and the cleanup's own error as
    ``_flextensor_cleanup_error``) so the caller can retry ``shutdown()``
    (loaders.py:1269-1286).
    """
    try:
        controller.shutdown()
    except BaseException as cleanup_error:
        LOGGER.warning("cleanup of a failed block build is incomplete", exc_info=True)
        try:
            primary.__dict__["_flextensor_cleanup_controller"] = controller
            primary.__dict__["_flextensor_cleanup_error"] = cleanup_error
            add_note = getattr(primary, "add_note", None)
            if callable(add_note):
                add_note(CLEANUP_NOTE)
        except BaseException:
            LOGGER.exception("could not attach the retryable cleanup handle to the primary error")


class _Released:
    """One packed-and-released source: the tensor object, its layout, a weak
    reference to the storage it viewed, and the host view holding its bytes."""

    __slots__ = ("source", "view", "size", "stride", "offset", "dtype", "device", "storage", "storage_nbytes")

    def __init__(self, source: torch.Tensor, view: torch.Tensor) -> None:
        storage = source.untyped_storage()
        self.source, self.view = source, view
        self.size, self.stride, self.offset = tuple(source.shape), source.stride(), source.storage_offset()
        self.dtype, self.device = source.dtype, source.device
        self.storage = StorageWeakRef(storage)  # weak: a released source must not keep its bytes alive
        self.storage_nbytes = storage.nbytes()


def _surviving(ref: StorageWeakRef) -> torch.UntypedStorage | None:
    """The storage behind ``ref`` if something else still holds it. Re-attaching
    through a weak reference is private torch API (``_new_with_weak_ptr``); where
    it is missing the source is restored into a new storage instead."""
    if ref.expired():
        return None
    attach = getattr(torch.UntypedStorage, "_new_with_weak_ptr", None)
    return attach(ref.cdata) if attach is not None else None


class _Rollback:
    """Puts packed-and-released sources back as they were when a build fails.

    A source whose original storage is still alive (another tensor, a parameter
    or a view's base aliases it) views that storage again at its own offset and
    strides; the bytes there were never touched. Sources whose storage died
    with the release get one new storage per original storage, of the original
    size, and their bytes are copied back from the host block at their own
    offsets and strides, so disjoint views of one storage share one storage
    again. The tensor objects are the same throughout (``.data`` is re-pointed).
    """

    def __init__(self) -> None:
        self._entries: list[_Released] = []

    def record(self, source: torch.Tensor, view: torch.Tensor) -> None:
        """Call before ``source`` is released."""
        self._entries.append(_Released(source, view))

    def restore(self) -> None:
        replacements: dict[StorageWeakRef, torch.UntypedStorage] = {}
        for e in self._entries:
            if e.source.numel() != 0 or math.prod(e.size) == 0:
                continue  # not released, or nothing to restore
            storage = _surviving(e.storage)
            if storage is not None:
                fill = False  # the original storage, whose bytes were never touched
            else:
                storage = replacements.get(e.storage)
                if storage is None:
                    storage = torch.empty(e.storage_nbytes, dtype=torch.uint8, device=e.device).untyped_storage()
                    replacements[e.storage] = storage
                fill = True
            restored = torch.empty(0, dtype=e.dtype, device=e.device)
            restored.set_(storage, e.offset, e.size, e.stride)
            if fill:
                dst, src = restored, e.view
                for d, st in enumerate(e.stride):  # an expanded source: write each element once
                    if st == 0 and e.size[d] > 1:
                        dst, src = dst.narrow(d, 0, 1), src.narrow(d, 0, 1)
                dst.copy_(src)
            e.source.data = restored
        self._entries.clear()

    def commit(self) -> None:
        self._entries.clear()


def _refuse_overlapping_sources(tensors_map: Mapping[int, torch.Tensor],
                                strategy_map: Mapping[str, Sequence[TensorStatistics]]) -> None:
    """Each source is packed on its own, so distinct tensors with overlapping bytes would stop aliasing:
    refuse them before any source is released (loaders.py:1217-1243). The check covers every tensor of
    ``tensors_map``, planned or not; disjoint views of one storage and repeated references to one tensor
    are fine."""
    managed = [tensors_map[i.tensor_id] for infos in strategy_map.values() for i in infos
               if i.tensor_id in tensors_map]
    groups = overlapping_views(managed, tensors_map.values())
    if groups:
        ids = {id(t): k for k, t in tensors_map.items()}
        shown = [sorted(ids.get(i, i) for i in g) for g in groups]
        raise ValueError("Block loaders cannot preserve distinct tensor views sharing storage with overlapping "
                         f"byte regions (tensor ids {shown}); give them separate storage (clone one)")


def _unique_tensors(strategy: Sequence[TensorStatistics], tensors_map: Mapping[int, torch.Tensor]):
    seen: set[int] = set()
    ids, tensors = [], []
    for info in strategy:
        if info.tensor_id in seen:
            continue
        seen.add(info.tensor_id)
        ids.append(info.tensor_id)
        tensors.append(tensors_map[info.tensor_id])
    return ids, tensors


class AllocationBlockController:
    def __init__(
        self,
        allocation_ordered: Mapping[int, Sequence[str]],
        device_gpu: torch.device,
        tensors_map: Mapping[int, torch.Tensor],
        strategy_map: Mapping[str, Sequence[TensorStatistics]],
        label_to_block_id: Mapping[str, int],
        *,
        host_pinner: HostPinner,
        release_tensor_memory: bool = True,
        copy_mode: int = nat.COPY_AUTO,
        copy_policy: nat.CopyPolicy | None = None,
        memory_alignment: int = 128,
        shm_block_name_map: Mapping[str, str] | None = None,
        load_from_shm: bool = False,
        encode_blocks: bool = False,
        hbm_encoded: Mapping[str, int] | None = None,
    ) -> None:
        """``shm_block_name_map`` puts each label's host block in a named shared-memory
        segment (loaders.py:1150-1175); with ``load_from_shm`` the segments already exist
        and are mapped instead of packed, and the tensors only supply their layouts.
        ``encode_blocks`` keeps an exponent-coded copy of each label's block, in the dense format
        (version 2), that saves at least a tenth of its bytes (:mod:`~flextensor_amd.expcode`); such a
        label's transfer is one decode launch that writes the raw block into its slot (no reference
        counterpart).
        ``hbm_encoded`` maps block keys of units kept resident in encoded form to the device bytes
        reserved for each encoded block: their slot group is packed into pageable host blocks (nothing
        crosses the link), each block is encoded into device memory in the dense format (version 2, decoded
        only from device memory), and :meth:`decode_resident`
        rebuilds it in its slot on the current stream (no reference counterpart)."""
        if load_from_shm and not shm_block_name_map:
            raise ValueError("load_from_shm needs shm_block_name_map")
        self.device_gpu = torch.device(device_gpu)
        self.host_pinner = host_pinner
        self.release_tensor_memory = release_tensor_memory
        self.copy_mode = copy_mode
        self.copy_policy = copy_policy
        self.shm_block_name_map = dict(shm_block_name_map or {})
        self.load_from_shm = load_from_shm
        self.block_map_cpu: dict[str, AllocationBlock] = {}
        self.label_to_cpu_tensor_id_map: dict[str, list[int]] = {}
        self.label_to_gpu_block: dict[str, AllocationBlock] = {}
        self.block_map_gpu: dict[int, torch.Tensor] = {}
        self.gpu_block_view_map: dict[str, torch.Tensor] = {}
        self.label_to_tensor_views_map: dict[str, list[torch.Tensor]] = {}
        self.tensor_id_to_view_map: dict[int, torch.Tensor] = {}
        self._gpu_slots: list[AllocationBlock] = []
        self.encoded: dict[str, Any] = {}  # label -> expcode.EncodedBlock
        self.use_encoded = True  # transfers of encoded labels decode (False: they copy the raw blocks)
        self.hbm_capacity = dict(hbm_encoded or {})
        self.hbm_encoded: dict[str, Any] = {}  # block key -> expcode.DeviceEncodedBlock
        self._rollback = _Rollback()
        _refuse_overlapping_sources(tensors_map, strategy_map)
        try:
            for _slot_id, labels in allocation_ordered.items():
                in_hbm = bool(labels) and all(x in self.hbm_capacity for x in labels)
                manager = AllocationManager(host_pinner=host_pinner, memory_alignment=memory_alignment,
                                            release_tensor_memory=False, pinned_memory=not in_hbm)
                for label in labels:
                    strategy = strategy_map.get(label, ())
                    if not strategy:
                        continue
                    ids, tensors = _unique_tensors(strategy, tensors_map)
                    shm_name = self.shm_block_name_map.get(label)
                    if self.shm_block_name_map and shm_name is None:
                        raise ValueError(f"no shared-memory block name for label {label!r}")
                    block = manager.block(shm_block_name=shm_name, load_from_shm=load_from_shm)
                    for t in tensors:
                        block.add(t)
                    views = block.allocate()
                    if release_tensor_memory:
                        for t, v in zip(tensors, views):
                            self._rollback.record(t, v)
                            t.data = torch.empty(0, dtype=t.dtype)
                    self.block_map_cpu[label] = block
                    self.label_to_cpu_tensor_id_map[label] = ids
                slot = manager.create_max_block(self.device_gpu)
                self._gpu_slots.append(slot)
                for label in labels:
                    self.label_to_gpu_block[label] = slot
            for label, block in self.block_map_cpu.items():
                views, prefix = block.project_views(self.label_to_gpu_block[label])
                self.label_to_tensor_views_map[label] = views
                self.block_map_gpu[label_to_block_id[label]] = prefix
                self.gpu_block_view_map[label] = prefix
            if self.hbm_capacity:
                from . import expcode

                for key, cap in self.hbm_capacity.items():
                    self.hbm_encoded[key] = expcode.DeviceEncodedBlock.from_raw(self.block_map_cpu[key].block, cap,
                                                                                self.device_gpu, dense=True)
            if encode_blocks:
                from . import expcode

                for label, block in self.block_map_cpu.items():
                    if label in self.hbm_capacity:
                        continue
                    enc = expcode.encode_if_smaller(block.block, dense=True)
                    if enc is not None:
                        self.encoded[label] = enc
            self.prepare_tensor_id_to_view_mapping()
        except BaseException as primary:
            # sources restored, segments this build created removed, maps cleared
            _cleanup_keeping_error(self, primary)
            raise

    def prepare_tensor_id_to_view_mapping(self) -> None:
        self.tensor_id_to_view_map = {}
        for label, views in self.label_to_tensor_views_map.items():
            for tid, view in zip(self.label_to_cpu_tensor_id_map[label], views):
                self.tensor_id_to_view_map[tid] = view

    def get_tensor_id_to_view_mapping(self) -> dict[int, torch.Tensor]:
        return self.tensor_id_to_view_map

    def cpu_views(self, label: str) -> list[torch.Tensor]:
        return self.block_map_cpu[label].views

    def schedule_transfer(self, label: str, non_blocking: bool = True) -> None:
        """One host-to-device copy of ``label``'s block into its slot, on the current stream: a decode
        launch for an encoded block (its workgroups hold the link at its peak, so the copy policy's grid
        does not apply), else a copy under this controller's copy policy."""
        enc = self.encoded.get(label) if self.use_encoded else None
        if enc is None:
            self.block_map_cpu[label].copy_to(self.gpu_block_view_map[label], non_blocking=non_blocking,
                                              mode=self.copy_mode, policy=self.copy_policy)
            return
        from .expcode import decode_h2d
        from .hip import current_stream

        dst = self.gpu_block_view_map[label]
        decode_h2d(dst, enc)
        if not non_blocking:
            current_stream(dst.device).synchronize()

    def decode_resident(self, key: str) -> None:
        """Rebuild the raw block of ``key`` (a unit kept encoded in HBM) in its slot, on the current
        stream."""
        self.hbm_encoded[key].decode(self.gpu_block_view_map[key])

    def transfer_bytes(self, label: str) -> int:
        """Bytes ``label``'s transfer writes into its slot (the raw block)."""
        return self.block_map_cpu[label].nbytes

    def refresh_encoded(self) -> None:
        """Re-encode every encoded block in place from its host block, after the host blocks were
        rewritten (a state-dict load). No transfer or decode may be in flight. A block whose new encoding
        outgrows its arena or reservation raises ValueError naming it."""
        for label, enc in self.encoded.items():
            try:
                enc.reencode(self.block_map_cpu[label].block)
            except ValueError as exc:
                raise ValueError(f"streamed unit block {label!r}: {exc}; release() and offload the model again "
                                 "(weights that do not shrink stream raw)") from exc
        for key, dev in self.hbm_encoded.items():
            try:
                dev.reencode(self.block_map_cpu[key].block)
            except ValueError as exc:
                raise ValueError(f"unit block {key!r} kept encoded in HBM: {exc}; release() and offload the "
                                 "model again to size the reservation for the new weights") from exc

    def link_bytes(self, label: str) -> int:
        """Bytes ``label``'s transfer reads over the host link: the encoded block when there is one."""
        enc = self.encoded.get(label) if self.use_encoded else None
        return enc.nbytes if enc is not None else self.block_map_cpu[label].nbytes

    def commit_construction(self) -> None:
        self._rollback.commit()

    def abort_construction(self, primary_error: BaseException | None = None) -> None:
        if primary_error is None:
            self.shutdown()
        else:
            _cleanup_keeping_error(self, primary_error)

    def _clear(self) -> None:
        self.encoded.clear()
        self.hbm_encoded.clear()
        for d in (self.block_map_cpu, self.label_to_cpu_tensor_id_map, self.label_to_gpu_block, self.block_map_gpu,
                  self.gpu_block_view_map, self.label_to_tensor_views_map, self.tensor_id_to_view_map):
            d.clear()
        self._gpu_slots = []

    def _release_shm_blocks(self) -> None:
        """Release every segment-backed block; raise the first failure after trying them all (retryable)."""
        first: BaseException | None = None
        for block in self.block_map_cpu.values():
            if block.shm_segment is not None:
                try:
                    block.release()  # the creator removes the segment's name; the mapping goes with its last view
                except BaseException as error:
                    first = first or error
        if first is not None:
            raise first

    def shutdown(self) -> None:
        self._rollback.restore()
        self._release_shm_blocks()
        self._clear()

    def release_gpu_blocks(self) -> None:
        self.label_to_gpu_block = {}
        self.block_map_gpu = {}
        self.gpu_block_view_map = {}
        self.label_to_tensor_views_map = {}
        self.tensor_id_to_view_map = {}
        self._gpu_slots = []
        self.hbm_encoded = {}

    def get_gpu_memory_bytes(self) -> int:
        """Ring slots, the slot units kept in HBM decode into, and their encoded blocks."""
        return sum(s.nbytes for s in self._gpu_slots) + sum(d.capacity for d in self.hbm_encoded.values())


class RawBlockController:
    def __init__(
        self,
        label_to_size_map: Mapping[str, int],
        block_sizes: Mapping[int, int],
        device_gpu: torch.device,
        tensors_map: Mapping[int, torch.Tensor],
        strategy_map: Mapping[str, Sequence[TensorStatistics]],
        label_to_block_id: Mapping[str, int],
        *,
        host_pinner: HostPinner,
        release_tensor_memory: bool = True,
        copy_mode: int = nat.COPY_AUTO,
        copy_policy: nat.CopyPolicy | None = None,
    ) -> None:
        self.device_gpu = torch.device(device_gpu)
        self.host_pinner = host_pinner
        self.release_tensor_memory = release_tensor_memory
        self.copy_mode = copy_mode
        self.copy_policy = copy_policy
        self.label_to_block_id = dict(label_to_block_id)
        self.block_map_cpu: dict[str, torch.Tensor] = {}
        self.block_meta_map: dict[str, list] = {}
        self.label_to_cpu_tensor_id_map: dict[str, list[int]] = {}
        self.block_map_gpu: dict[int, torch.Tensor] = {}
        self.gpu_block_view_map: dict[str, torch.Tensor] = {}
        self.label_to_tensor_views_map: dict[str, list[torch.Tensor]] = {}
        self.tensor_id_to_view_map: dict[int, torch.Tensor] = {}
        self._rollback = _Rollback()
        _refuse_overlapping_sources(tensors_map, strategy_map)
        try:
            # device slots first: a failed allocation then leaves every source untouched
            self.block_map_gpu = {
                b: torch.zeros(max(n, 1), dtype=torch.uint8, device=self.device_gpu) for b, n in block_sizes.items()
            }
            for label, strategy in strategy_map.items():
                if not strategy:
                    continue
                ids, tensors = _unique_tensors(strategy, tensors_map)
                block = host_pinner.new_block(label_to_size_map[label])
                block.zero_()
                self.block_map_cpu[label] = block
                self.block_meta_map[label] = self.combine_tensors(tensors, block)
                self.label_to_cpu_tensor_id_map[label] = ids
            self.gpu_block_view_map = {
                label: self.block_map_gpu[b][: self.block_map_cpu[label].numel()]
                for label, b in self.label_to_block_id.items()
                if label in self.block_map_cpu
            }
            self.prepare_tensor_id_to_view_mapping()
        except BaseException as primary:
            _cleanup_keeping_error(self, primary)
            raise

    def combine_tensors(self, tensors: Sequence[torch.Tensor], combined: torch.Tensor) -> list:
        """Pack back to back; metadata per tensor is (start, end, shape, dtype, stride)."""
        meta = []
        cursor = 0
        for t in tensors:
            n = t.numel() * t.element_size()
            if is_dense_layout(t):
                stride = tuple(t.stride())
                src = raw_storage_bytes(t.detach()) if t.numel() else torch.empty(0, dtype=torch.uint8)
            else:
                c = t.detach().contiguous()
                stride = contiguous_strides(c.shape)
                src = c.view(-1).view(torch.uint8)
            combined[cursor: cursor + n] = src
            meta.append((cursor, cursor + n, tuple(t.shape), t.dtype, stride))
            if self.release_tensor_memory:
                rollback = getattr(self, "_rollback", None)
                if rollback is not None:
                    rollback.record(t, view_from_block(combined, t.dtype, tuple(t.shape), cursor, stride))
                t.data = torch.empty(0, dtype=t.dtype)
            cursor += n
        return meta

    @staticmethod
    def reconstruct_original_shapes(combined: torch.Tensor, metadata: Sequence) -> list[torch.Tensor]:
        return [view_from_block(combined, dtype, shape, start, stride) for start, _end, shape, dtype, stride in metadata]

    def prepare_tensor_id_to_view_mapping(self) -> None:
        self.label_to_tensor_views_map = {
            label: self.reconstruct_original_shapes(self.block_map_gpu[self.label_to_block_id[label]], meta)
            for label, meta in self.block_meta_map.items()
        }
        self.tensor_id_to_view_map = {}
        for label, views in self.label_to_tensor_views_map.items():
            for tid, v in zip(self.label_to_cpu_tensor_id_map[label], views):
                self.tensor_id_to_view_map[tid] = v

    def get_tensor_id_to_view_mapping(self) -> dict[int, torch.Tensor]:
        return self.tensor_id_to_view_map

    def schedule_transfer(self, label: str, non_blocking: bool = True) -> None:
        from .hip import copy_h2d, current_stream

        dst = self.gpu_block_view_map[label]
        copy_h2d(dst, self.block_map_cpu[label], self.copy_mode, policy=self.copy_policy)
        if not non_blocking:
            current_stream(dst.device).synchronize()

    def transfer_bytes(self, label: str) -> int:
        return self.block_map_cpu[label].numel()

    def commit_construction(self) -> None:
        self._rollback.commit()

    def abort_construction(self, primary_error: BaseException | None = None) -> None:
        if primary_error is None:
            self.shutdown()
        else:
            _cleanup_keeping_error(self, primary_error)

    def shutdown(self) -> None:
        self._rollback.restore()
        for d in (self.block_map_cpu, self.block_meta_map, self.label_to_cpu_tensor_id_map, self.block_map_gpu,
                  self.gpu_block_view_map, self.label_to_tensor_views_map, self.tensor_id_to_view_map):
            d.clear()

    def release_gpu_blocks(self) -> None:
        self.block_map_gpu = {}
        self.gpu_block_view_map = {}
        self.label_to_tensor_views_map = {}
        self.tensor_id_to_view_map = {}

    def get_gpu_memory_bytes(self) -> int:
        return sum(b.numel() for b in self.block_map_gpu.values())


def describe(controller: Any) -> str:
    labels = list(getattr(controller, "block_map_cpu", {}))
    return f"{type(controller).__name__}(labels={len(labels)}, gpu_bytes={controller.get_gpu_memory_bytes()})"
