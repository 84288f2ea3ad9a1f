"""Re-measuring a streaming plan in flight (``request_strategy_replan``), on the CPU.

The reference's replan re-measures units after the compute changed under a
running offload and rebuilds its strategy (offload_manager.py:667-720,
1294-1325; compile/replan_status.py, whose status vocabulary these tests
check). Here what depends on compute times is the ring's copy engine, so a
replan that measures a compute-bound pass must move a link-bound manager's
ring copies back to the per-size policy, and the reverse. The managers run on
the host with their ring slots on the CPU, their loaders on recording fake
streams, and the replan's collector on scripted timing events.
"""

from __future__ import annotations

import functools
import logging
from unittest import mock

import pytest
import torch

import flextensor_amd.manager as M
from flextensor_amd import link_model as L
from flextensor_amd.config import OffloadConfig
from flextensor_amd.replan import (REPLAN_MEASURE_PASSES, REPLAN_WARMUP_PASSES, StrategyReplanStatus,
                                   measured_compute, replanned_link)
from flextensor_amd.timing import OffloadTimingCollector, OffloadTimingSnapshot, TrapTimingRecord
from tests.fakes import FakeBackend, Recorder


class _Stack(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList(torch.nn.Linear(4, 4) for _ in range(3))


def _fake_link(kernel_faster_up_to: int = 1 << 20) -> L.LinkMeasurement:
    sizes = L.link_probe_sizes(1 << 28)
    sdma = L.CopyCurve("sdma", {n: 0.01 + n / 50e6 for n in sizes})
    kernel = L.CopyCurve("kernel", {n: (sdma.best_ms[n] / 1.3 if n <= kernel_faster_up_to else sdma.best_ms[n] * 1.02)
                                    for n in sizes})
    km, sm, ns = L.choose_copy_policy(sdma, kernel)
    return L.LinkMeasurement(sdma, kernel, km, sm, ns)


class _ScriptedEvent:
    """A timing event whose role (transfer, compute or wait, start or end) is its creation order within a
    label's six events, as the collector creates them; compute spans last ``compute_ms[0]``."""

    def __init__(self, role: int, compute_ms: list[float]) -> None:
        self.role, self.compute_ms = role, compute_ms

    def record(self, stream=None) -> "_ScriptedEvent":
        return self

    def elapsed_time(self, end: "_ScriptedEvent") -> float:
        return self.compute_ms[0] if self.role == 2 else 0.05


def _scripted_collector(labels, compute_ms: list[float]) -> OffloadTimingCollector:
    made = []

    def factory():
        made.append(None)
        return _ScriptedEvent((len(made) - 1) % 6, compute_ms)

    return OffloadTimingCollector(labels, event_factory=factory, current_stream=lambda: None,
                                  synchronize=lambda: None, is_capturing=lambda: False, log_every=0)


@pytest.fixture
def streaming():
    """Managers in INFERENCE on the host: ring slots on the CPU, loaders on fake streams, a fake link."""
    made = []
    rec = Recorder()
    loaders = {cls: functools.partial(getattr(M, cls), backend=FakeBackend(rec))
               for cls in ("PreallocatedBatchTransferTensorLoader", "PreallocatedBatchTransferTensorLoaderReordered")}
    with mock.patch.object(M.nat, "load", lambda: None), \
            mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", lambda self, ts: 0), \
            mock.patch.object(M, "measure_link", lambda sizes, dev: _fake_link()), \
            mock.patch.multiple(M, **loaders), \
            mock.patch.object(M.hip, "is_capturing", lambda: False):
        def run(name, profiled_ms, **cfg):
            made.append(name)
            mgr = M.get_offload_manager(name)
            mgr.offload(_Stack(), OffloadConfig(include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1,
                                                pinned_memory=False, **{"max_inflight_passes": 0, **cfg}))
            mgr.device = torch.device("cpu")
            mgr.order = [u.label for u in mgr.units]
            mgr.durations = {x: [profiled_ms] for x in mgr.order}
            mgr._to_inference()
            assert mgr.phase == M.OffloadPhase.INFERENCE
            return mgr

        def one_pass(mgr):
            for label in mgr.order:
                mgr.loader.enter(label)
                mgr.loader.exit(label)
            mgr._after_forward()

        yield run, one_pass
    for n in made:
        M._MANAGERS.pop(n, None)


def test_measured_compute_takes_each_units_median():
    snaps = [OffloadTimingSnapshot([TrapTimingRecord("a", 1.0, c, 0.0), TrapTimingRecord("b", 0.0, 2 * c, 0.0)])
             for c in (1.0, 3.0, 2.0)]
    assert measured_compute(snaps, ["a", "b", "c"]) == {"a": 2.0, "b": 4.0}  # c was never timed
    zero = [OffloadTimingSnapshot([TrapTimingRecord("a", 1.0, 0.0, 0.0)])]
    assert measured_compute(zero, ["a"]) == {}  # an untimed unit is not a zero-cost unit


def test_replanned_link_follows_the_pass_rule():
    link = _fake_link()
    sizes = [64 << 20] * 4
    transfer = link.transfer_ms(sizes)
    fast = replanned_link(link, 0.1 * transfer, sizes)
    assert fast.link_bound and fast.kernel_grid == L.RING_KERNEL_GRID and fast.kernel_max_bytes >= max(sizes)
    slow = replanned_link(fast, 3.0 * transfer, sizes)  # from a link-bound policy back to the measured one
    assert not slow.link_bound and slow.kernel_grid == 0
    assert slow.policy() == L.choose_copy_policy(link.sdma, link.kernel)
    assert (slow.pass_compute_ms, slow.source) == (3.0 * transfer, "replan")
    assert slow.pass_transfer_ms == pytest.approx(transfer)
    assert slow.sdma is link.sdma  # the measured curves stay the link model


def test_a_compute_bound_replan_moves_a_link_bound_ring_back_to_the_measured_policy(streaming):
    run, one_pass = streaming
    mgr = run("replan-down", 1e-6)
    assert mgr.link.link_bound and mgr.controller.copy_policy.kernel_grid == L.RING_KERNEL_GRID
    assert mgr.loader.link_bound  # a link-bound ring waits for its copies on the host
    assert mgr.strategy_replan_status == StrategyReplanStatus("idle", True, None)
    compute = [1e6]
    with mock.patch.object(mgr, "_new_replan_collector", lambda: _scripted_collector(mgr.order, compute)):
        kept = mgr.loader.offload_timing_collector
        passes = mgr.request_strategy_replan()
    assert passes == REPLAN_WARMUP_PASSES + REPLAN_MEASURE_PASSES
    assert mgr.strategy_replan_status == StrategyReplanStatus("in_progress", False, None)
    assert mgr.loader.offload_timing_collector is not kept
    for _ in range(passes - 1):
        one_pass(mgr)
        assert mgr.strategy_replan_status.state == "in_progress"
    one_pass(mgr)
    assert mgr.strategy_replan_status == StrategyReplanStatus("done", True, True)
    assert mgr.loader.offload_timing_collector is kept  # the caller's timing is back in place
    assert mgr.durations == {x: [1e6] for x in mgr.order}
    assert not mgr.link.link_bound and mgr.link.source == "replan"
    assert mgr.link.pass_compute_ms == pytest.approx(1e6 * len(mgr.order))
    assert mgr.controller.copy_policy == mgr.link.native_policy() and mgr.controller.copy_policy.kernel_grid == 0
    assert not mgr.loader.link_bound  # a compute-bound one on the compute stream, so the host runs ahead
    # and back: a link-bound replan gives the ring the kernel again
    compute[0] = 1e-6
    with mock.patch.object(mgr, "_new_replan_collector", lambda: _scripted_collector(mgr.order, compute)):
        for _ in range(mgr.request_strategy_replan()):
            one_pass(mgr)
    assert mgr.link.link_bound and mgr.controller.copy_policy.kernel_grid == L.RING_KERNEL_GRID
    assert mgr.loader.link_bound
    assert mgr.strategy_replan_status == StrategyReplanStatus("done", True, True)


def test_requests_that_cannot_start_warn_and_return_zero(streaming, caplog):
    run, one_pass = streaming
    mgr = run("replan-refuse", 1e-6)
    with mock.patch.object(mgr, "_new_replan_collector", lambda: _scripted_collector(mgr.order, [1.0])), \
            caplog.at_level(logging.WARNING, logger="flextensor_amd.manager"):
        assert mgr.request_strategy_replan() == 3
        assert mgr.request_strategy_replan() == 0  # one in flight
        assert "already in flight" in caplog.text
        caplog.clear()
        for _ in range(3):
            one_pass(mgr)
        # graph replays need the replay-timing mode the graph was captured with
        assert mgr.request_strategy_replan(manual_update_state=True) == 0
        assert "offload_timing='cuda_graph'" in caplog.text
    assert M.request_strategy_replan("replan-refuse", manual_update_state=True) == 0
    fresh = M.get_offload_manager("replan-fresh")
    try:
        fresh.offload(_Stack(), OffloadConfig(include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1))
        with caplog.at_level(logging.WARNING, logger="flextensor_amd.manager"):
            assert fresh.request_strategy_replan() == 0
        assert "reach inference first" in caplog.text
        assert fresh.strategy_replan_status == StrategyReplanStatus("idle", False, None)
    finally:
        M._MANAGERS.pop("replan-fresh", None)


def test_without_a_link_measurement_the_replan_keeps_the_plan(streaming):
    """With no measured link (a pinned copy engine) nothing in the plan depends on compute times: the replan
    stores the new durations and reports applied=False."""
    run, one_pass = streaming
    mgr = run("replan-keep", 1.0, copy_engine="sdma", link_benchmark=False)
    assert mgr.link is None and not mgr.loader.link_bound
    policy = mgr.controller.copy_policy
    with mock.patch.object(mgr, "_new_replan_collector", lambda: _scripted_collector(mgr.order, [7.0])):
        for _ in range(mgr.request_strategy_replan()):
            one_pass(mgr)
    assert mgr.strategy_replan_status == StrategyReplanStatus("done", True, False)
    assert mgr.durations == {x: [7.0] for x in mgr.order} and mgr.controller.copy_policy is policy


def test_a_failed_rebuild_reports_failed_and_refuses_more(streaming, caplog):
    run, one_pass = streaming
    mgr = run("replan-fail", 1e-6)
    with mock.patch.object(mgr, "_new_replan_collector", lambda: _scripted_collector(mgr.order, [1.0])), \
            mock.patch.object(M, "replanned_link", side_effect=RuntimeError("rebuild broke")):
        kept = mgr.loader.offload_timing_collector
        n = mgr.request_strategy_replan()
        for _ in range(n - 1):
            one_pass(mgr)
        with pytest.raises(RuntimeError, match="rebuild broke"), \
                caplog.at_level(logging.ERROR, logger="flextensor_amd.manager"):
            one_pass(mgr)
    assert mgr.strategy_replan_status == StrategyReplanStatus("failed", False, False)
    assert mgr.loader.offload_timing_collector is kept
    assert mgr.request_strategy_replan() == 0
