"""The copy engine a measured pass chooses, per manager, on the GPU.

A pass whose profiled compute is far below its transfer time (an 8-layer
4096 -> 11008 -> 4096 MLP stack at 16 rows) is link-bound: its ring copies
go to the zero-copy kernel at the ring grid. The same stack at 32768 rows
computes for about three times its transfer time and keeps the measured
per-size policy (SDMA for the 180 MB layers).

The link-bound manager also waits for its ring copies on the host rather
than on the compute stream.

Both managers live in one process and stream in alternation, as the
reference's named managers do (offload_manager.py:2817-2850): each
controller carries its own policy into every copy, the library's
process-wide default is never changed, and both stream outputs bitwise equal
to the resident forward.
"""

from __future__ import annotations

import pytest
import torch

from flextensor_amd import _native as nat
from flextensor_amd import link_model as L
from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager

pytestmark = pytest.mark.gpu


def test_link_bound_and_compute_bound_managers_stream_side_by_side(gpu):
    nat.load()
    default = nat.get_copy_policy()
    dev = gpu
    rows = {"link-bound-gpu": 16, "compute-bound-gpu": 32768}
    models, inputs, want, managers = {}, {}, {}, {}
    for name, m in rows.items():
        models[name] = W.build_mlp_stack(8, 4096, 11008, seed=0)
        inputs[name] = W.mlp_input(m, 4096, seed=0).to(dev)
        with torch.no_grad():
            want[name] = W.build_mlp_stack(8, 4096, 11008, seed=0).to(dev)(inputs[name])
    torch.cuda.empty_cache()
    try:
        for name in rows:
            managers[name] = OffloadManager(name)
            managers[name].offload(models[name], OffloadConfig(include_patterns=["layers.*"], num_blocks=2,
                                                               min_blocks=2, discovery_iters=1, profiling_iters=1))
        got = {}
        with torch.no_grad():
            for _ in range(4):  # discovery, profiling, then two streamed passes, alternating managers
                for name in rows:
                    got[name] = models[name](inputs[name])
        torch.cuda.synchronize()
        link_bound, compute_bound = managers["link-bound-gpu"], managers["compute-bound-gpu"]
        unit_bytes = max(link_bound._unit(u).nbytes for u in link_bound.plan.streamed)
        assert link_bound.link is not None and link_bound.link.source == "measured"
        assert link_bound.link.link_bound and link_bound.link.kernel_grid == L.RING_KERNEL_GRID
        pol = link_bound.controller.copy_policy
        assert pol.kernel_max_bytes >= unit_bytes and pol.kernel_grid == L.RING_KERNEL_GRID
        assert compute_bound.link is not None and not compute_bound.link.link_bound
        pol = compute_bound.controller.copy_policy
        assert pol.kernel_max_bytes < unit_bytes and pol.kernel_grid == 0
        assert nat.get_copy_policy() == default  # neither manager touched the process-wide default
        # the link-bound ring waits for its copies on the host, the compute-bound one on the compute stream
        assert link_bound.loader.link_bound and not compute_bound.loader.link_bound
        for name in rows:
            assert torch.equal(got[name], want[name]), name
        # one manager goes; the other keeps streaming bitwise under its own policy
        managers.pop("link-bound-gpu").release(preserve_model=False)
        with torch.no_grad():
            again = models["compute-bound-gpu"](inputs["compute-bound-gpu"])
        assert torch.equal(again, want["compute-bound-gpu"])
        assert nat.get_copy_policy() == default
    finally:
        for mgr in managers.values():
            mgr.release(preserve_model=False)
        torch.cuda.empty_cache()


def test_a_replan_follows_the_workload_when_the_batch_changes(gpu):
    """``request_strategy_replan`` (offload_manager.py:1294-1325) on the GPU. A stack profiled at 16 rows
    is link-bound and copies its ring with the zero-copy kernel. Fed 32768-row batches it computes for
    longer than its transfers, and a replan measured on those passes moves the ring back to the measured
    per-size policy (SDMA for the 180 MB layers). Back at 16 rows, a second replan returns to the kernel.
    A 1 GB budget keeps some layers resident, so the reordered loader runs and its ring waits follow the
    policy: on the host while link-bound, on the compute stream otherwise. Every pass is bitwise equal to
    the resident forward."""
    import flextensor_amd as ft

    nat.load()
    default = nat.get_copy_policy()
    model = W.build_mlp_stack(8, 4096, 11008, seed=0)
    resident = W.build_mlp_stack(8, 4096, 11008, seed=0).to(gpu)
    small, large = (W.mlp_input(m, 4096, seed=0).to(gpu) for m in (16, 32768))
    with torch.no_grad():
        want = {16: resident(small), 32768: resident(large)}
    del resident
    torch.cuda.empty_cache()
    mgr = OffloadManager("replan-gpu")
    mgr.offload(model, OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                                     profiling_iters=1, max_gpu_mem_bytes=1_000_000_000))
    try:
        assert mgr.strategy_replan_status == ft.StrategyReplanStatus("idle", False, None)
        with torch.no_grad():
            for _ in range(3):  # discovery, profiling at 16 rows, one streamed pass
                got = model(small)
        assert torch.equal(got, want[16])
        assert mgr.plan.resident and mgr.plan.reordered
        assert mgr.link.link_bound and mgr.controller.copy_policy.kernel_grid == L.RING_KERNEL_GRID
        assert mgr.loader.link_bound
        assert mgr.strategy_replan_status.can_request
        for rows, x, link_bound in ((32768, large, False), (16, small, True)):
            print(f"replan at {rows} rows", flush=True)
            n = mgr.request_strategy_replan()
            assert n > 0 and mgr.strategy_replan_status.state == "in_progress"
            with torch.no_grad():
                for _ in range(n):
                    got = model(x)
                    assert torch.equal(got, want[rows])
            status = mgr.strategy_replan_status
            assert status == ft.StrategyReplanStatus("done", True, True), status
            assert mgr.link.link_bound == link_bound and mgr.link.source == "replan", mgr.link.describe()
            assert mgr.controller.copy_policy == mgr.link.native_policy()
            assert mgr.loader.link_bound == link_bound
            with torch.no_grad():
                assert torch.equal(model(x), want[rows])  # streaming under the new policy
        assert nat.get_copy_policy() == default
    finally:
        mgr.release(preserve_model=False)
        torch.cuda.empty_cache()
