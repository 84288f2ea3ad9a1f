"""Pipelined block loaders: the per-label hot loop (row a8 of the hot path).

Both loaders keep the reference's operation order exactly, because the
order is what makes the pipeline correct:

* :class:`PreallocatedBatchTransferTensorLoader` (loaders.py:1473-1658):
  ``enter(L)`` submits the transfer scheduled at ``L`` into
  ``label_to_block_id[L]``; ``exit(L)`` makes the compute stream wait for
  that transfer (whose bytes the next label reads) and records the last use
  of every slot ``L`` consumed; the last label joins the transfer stream.
* :class:`PreallocatedBatchTransferTensorLoaderReordered` (loaders.py:1661-1858):
  ``enter(L)`` first waits for every transfer whose consumer is ``L``, then
  submits; ``exit(L)`` only releases slots. This lets a transfer be issued
  several labels before its consumer (rearranged schedules).

If a pass aborted mid-way, the first label's ``enter`` joins the still-active
runtime and drops stale tickets (loaders.py:1538-1551). Transfers whose
consumer runs earlier in the pass are issued once at construction
(``preload``) and then every pass by the label that schedules them.
"""

from __future__ import annotations

import logging
from collections.abc import Mapping, Sequence
from functools import partial
from typing import Any

from .planner import LayerStatistics, find_transfers_for_preload
from .prefetch_policy import PiecewisePrefetchPolicy, PiecewisePrefetchPolicyError
from .timing import OffloadTimingCollector
from .transfer import HipTransferRuntime, StreamBackend, TransferTicket

LOGGER = logging.getLogger(__name__)


def compute_to_block_ids(label_to_block_id: Mapping[str, int], t2c: Mapping[str, str]) -> dict[str, list[int]]:
    """Compute label -> slots it reads (the slots filled by transfers it consumes)."""
    out: dict[str, list[int]] = {}
    for transfer, compute in t2c.items():
        out.setdefault(compute, []).append(label_to_block_id[transfer])
    return out


class Loader:
    def enter(self, label: str) -> None:
        raise NotImplementedError

    def exit(self, label: str) -> None:
        raise NotImplementedError

    def shutdown(self) -> None:
        return None


class PreallocatedLoader(Loader):
    def __init__(self, allocation_controller: Any, offload_timing_collector: OffloadTimingCollector | None = None,
                 piecewise_prefetch_policy: PiecewisePrefetchPolicy | None = None) -> None:
        self.allocation_controller = allocation_controller
        self.offload_timing_collector = offload_timing_collector or OffloadTimingCollector(enabled=False)
        self.piecewise_prefetch_policy = piecewise_prefetch_policy or PiecewisePrefetchPolicy()

    def preload(self) -> None:
        raise NotImplementedError

    def prepare(self) -> None:
        self.preload()

    def sync_prev_onload(self) -> None:
        raise NotImplementedError

    def join_after_forward(self) -> None:
        raise NotImplementedError

    def release_memory(self) -> None:
        return None

    def shutdown(self) -> None:
        self.allocation_controller.shutdown()

    def get_gpu_memory_bytes(self) -> int:
        return self.allocation_controller.get_gpu_memory_bytes()


class _PipelinedLoader(PreallocatedLoader):
    """State and lifecycle shared by both loaders."""

    def __init__(
        self,
        layer_stats: Sequence[LayerStatistics],
        device_gpu: Any,
        label_to_block_id: Mapping[str, int],
        transfer_to_compute_map: Mapping[str, str],
        allocation_controller: Any,
        offload_timing_collector: OffloadTimingCollector | None = None,
        piecewise_prefetch_policy: PiecewisePrefetchPolicy | None = None,
        backend: StreamBackend | None = None,
    ) -> None:
        super().__init__(allocation_controller, offload_timing_collector, piecewise_prefetch_policy)
        self.device_gpu = device_gpu
        self.label_to_block_id = dict(label_to_block_id)
        self.transfer_to_compute_map = dict(transfer_to_compute_map)
        self._transfer_runtime = HipTransferRuntime(device_gpu, backend=backend)
        self.backend = self._transfer_runtime.backend
        self.transfer_stream = self._transfer_runtime.transfer_stream
        self._compute_to_block_ids = compute_to_block_ids(self.label_to_block_id, self.transfer_to_compute_map)
        self.first_layer_label = layer_stats[0].label if layer_stats else None
        self.last_layer_label = layer_stats[-1].label if layer_stats else None
        self.preload_transfers = find_transfers_for_preload(self.transfer_to_compute_map, layer_stats)
        # The pass waits on the link (the manager sets it for link-bound passes). Each loader then orders
        # its waits for that: the reordered loader waits for ring copies on the host, the default loader
        # releases the slots a label read before it waits (see their enter and exit). Graph capture keeps
        # the reference's order.
        self.link_bound = False

    def _trace(self, label: str) -> str:
        return f"schedule={label} consume={self.transfer_to_compute_map[label]}"

    def sync_prev_onload(self) -> None:
        self.backend.current_stream().wait_stream(self.transfer_stream)

    def _start_pass_if_first(self, label: str) -> None:
        if label != self.first_layer_label:
            return
        if self._transfer_runtime.is_active:
            LOGGER.debug("%s: abort recovery - joining the transfer stream and dropping %d scheduled entries",
                         type(self).__name__, len(self.scheduled_transfers))
            self._transfer_runtime.join()
            self.scheduled_transfers.clear()
            # The aborted pass never reached the labels that load the next pass's first slots:
            # load them again, as at construction. (The reference, loaders.py:1729-1740, only
            # joins and clears, so its first labels would then read stale slots.)
            self.preload()
        self.offload_timing_collector.on_pass_start()
        self.piecewise_prefetch_policy.reset()

    def _release_slots(self, label: str) -> None:
        slots = self._compute_to_block_ids.get(label)
        if self._transfer_runtime.is_active and slots:
            for slot in slots:
                self._transfer_runtime.finish_use(slot)
        else:
            # keeps one compute-stream event per label, as the reference does
            self.backend.current_stream().record_event()

    def _end_pass_if_last(self, label: str) -> None:
        if label != self.last_layer_label:
            return
        if self._transfer_runtime.is_active:
            self._transfer_runtime.join()
        error: BaseException | None = None
        try:
            self.piecewise_prefetch_policy.on_piece_join(at_last_layer=True)
        except PiecewisePrefetchPolicyError as exc:
            error = exc
        self.scheduled_transfers.clear()
        if error is not None:
            raise error

    def join_after_forward(self) -> None:
        error: BaseException | None = None
        try:
            self.piecewise_prefetch_policy.on_piece_join(at_last_layer=False)
        except PiecewisePrefetchPolicyError as exc:
            error = exc
        self._transfer_runtime.join()
        self.scheduled_transfers.clear()
        if error is not None:
            raise error

    def shutdown(self) -> None:
        self._transfer_runtime.close()
        super().shutdown()


class PreallocatedBatchTransferTensorLoader(_PipelinedLoader):
    def __init__(self, *args: Any, **kwargs: Any) -> None:
        super().__init__(*args, **kwargs)
        self.scheduled_transfers: dict[str, TransferTicket] = {}
        self.prepare()

    def preload(self) -> None:
        if not self.preload_transfers:
            return
        rt = self._transfer_runtime
        rt.begin()
        for label in self.preload_transfers:
            rt.submit(self.label_to_block_id[label], partial(self.allocation_controller.schedule_transfer, label),
                      trace_label=self._trace(label))
        rt.join()

    def enter(self, label: str) -> None:
        tc, pp, rt = self.offload_timing_collector, self.piecewise_prefetch_policy, self._transfer_runtime
        self._start_pass_if_first(label)
        if not rt.is_active:
            rt.begin()
        if label not in self.label_to_block_id:
            tc.record_compute_start(label)
            return

        def transfer() -> None:
            tc.record_transfer_start(label, self.transfer_stream)
            self.allocation_controller.schedule_transfer(label)

        self.scheduled_transfers[label] = rt.submit(self.label_to_block_id[label], transfer,
                                                    trace_label=self._trace(label))
        pp.on_schedule(schedule_label=label, compute_label=label)
        tc.record_transfer_end(label, self.transfer_stream)
        tc.record_compute_start(label)

    def exit(self, label: str) -> None:
        tc, pp = self.offload_timing_collector, self.piecewise_prefetch_policy
        tc.record_compute_end(label)  # before the wait: compute_ms excludes stalls
        # link-bound: the slots this label read are released before the wait for the next transfer, so
        # the transfer after it (into one of those slots) can queue behind it instead of waiting for it
        early = self.link_bound and not self.backend.is_capturing()
        if early:
            self._release_slots(label)
        ticket = self.scheduled_transfers.get(label)
        if ticket is not None:
            tc.record_wait_start(label)
            self._transfer_runtime.wait_ready(ticket)
            pp.on_wait(label)
            tc.record_wait_end(label)
        if not early:
            self._release_slots(label)
        self._end_pass_if_last(label)


class PreallocatedBatchTransferTensorLoaderReordered(_PipelinedLoader):
    def __init__(self, *args: Any, **kwargs: Any) -> None:
        super().__init__(*args, **kwargs)
        self.scheduled_transfers: dict[str, list[TransferTicket]] = {}
        self._preloaded_compute_labels: set[str] = set()
        self.prepare()

    def preload(self) -> None:
        if not self.preload_transfers:
            return
        rt = self._transfer_runtime
        rt.begin()
        for label, compute in self.preload_transfers.items():
            rt.submit(self.label_to_block_id[label], partial(self.allocation_controller.schedule_transfer, label),
                      trace_label=f"schedule={label} consume={compute}")
            self._preloaded_compute_labels.add(compute)
        rt.join()

    def enter(self, label: str) -> None:
        """Wait for the transfers ``label`` consumes, then submit the one scheduled at ``label``.

        With ``link_bound`` (link-bound passes) the host blocks on each
        transfer instead of the compute stream waiting on it, and the
        transfer scheduled at ``label`` is submitted before that block, so
        the transfer stream already holds the next copy while the host
        waits and the link never waits on the host. The slot it fills is
        never one ``label`` consumes (those stay busy until ``exit``), so
        the two orders fill the same slots. Graph capture keeps the
        reference's order and stream waits.
        """
        tc, pp, rt = self.offload_timing_collector, self.piecewise_prefetch_policy, self._transfer_runtime
        self._start_pass_if_first(label)
        if not rt.is_active:
            rt.begin()
        if label in self._preloaded_compute_labels:
            pp.on_wait(label)
        host = self.link_bound and not self.backend.is_capturing()
        ahead = host and label in self.label_to_block_id and self.transfer_to_compute_map[label] != label
        if ahead:
            self._submit(label)
        tickets = self.scheduled_transfers.pop(label, None)
        if tickets:
            tc.record_wait_start(label)
            for ticket in tickets:
                rt.wait_ready(ticket, host=host)
            pp.on_wait(label)
            tc.record_wait_end(label)
        if label not in self.label_to_block_id:
            tc.record_compute_start(label)
            return
        if not ahead:
            self._submit(label)
        tc.record_compute_start(label)

    def _submit(self, label: str) -> None:
        tc, pp, rt = self.offload_timing_collector, self.piecewise_prefetch_policy, self._transfer_runtime
        compute = self.transfer_to_compute_map[label]

        def transfer() -> None:
            tc.record_transfer_start(label, self.transfer_stream)
            self.allocation_controller.schedule_transfer(label)

        ticket = rt.submit(self.label_to_block_id[label], transfer, trace_label=f"schedule={label} consume={compute}")
        tc.record_transfer_end(label, self.transfer_stream)
        self.scheduled_transfers.setdefault(compute, []).append(ticket)
        pp.on_schedule(schedule_label=label, compute_label=compute)

    def exit(self, label: str) -> None:
        self.offload_timing_collector.record_compute_end(label)
        self._release_slots(label)
        self._end_pass_if_last(label)
