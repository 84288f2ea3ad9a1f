"""The copy engine a measured pass chooses, on the GPU.

A pass whose profiled compute is far below its transfer time (an 8-layer
4096 -> 11008 -> 4096 MLP stack at 16 rows) is link-bound: its ring copies
go to the zero-copy kernel at the ring grid. The same stack at 32768 rows
computes for about three times its transfer time and keeps the measured
per-size policy (SDMA for the 180 MB layers). Both stream outputs bitwise
equal to the resident forward, so the kernel copies move the same bytes.
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


@pytest.fixture
def keep_policy():
    nat.load()
    before = nat.get_copy_policy()
    yield
    nat.set_copy_policy(*before)


def _streamed_vs_resident(rows: int, name: str):
    dev = torch.device("cuda", 0)
    model = W.build_mlp_stack(8, 4096, 11008, seed=0)
    x = W.mlp_input(rows, 4096, seed=0).to(dev)
    with torch.no_grad():
        want = W.build_mlp_stack(8, 4096, 11008, seed=0).to(dev)(x)
    mgr = OffloadManager(name)
    mgr.offload(model, OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2,
                                     discovery_iters=1, profiling_iters=1))
    try:
        with torch.no_grad():
            for _ in range(4):  # discovery, profiling, then two streamed passes
                got = model(x)
        torch.cuda.synchronize()
        unit_bytes = max(mgr._unit(u).nbytes for u in mgr.plan.streamed)
        return mgr.link, nat.get_copy_policy(), unit_bytes, bool(torch.equal(got, want))
    finally:
        mgr.release(preserve_model=False)
        torch.cuda.empty_cache()


def test_a_link_bound_pass_copies_its_slots_with_the_kernel(keep_policy):
    link, policy, unit_bytes, same = _streamed_vs_resident(16, "link-bound-gpu")
    assert link is not None and link.source == "measured"
    assert link.link_bound and link.kernel_grid == L.RING_KERNEL_GRID
    assert policy[0] >= unit_bytes and policy[3] == L.RING_KERNEL_GRID
    assert same


def test_a_compute_bound_pass_keeps_sdma_for_its_slots(keep_policy):
    link, policy, unit_bytes, same = _streamed_vs_resident(32768, "compute-bound-gpu")
    assert link is not None and not link.link_bound and link.kernel_grid == 0
    assert policy[0] < unit_bytes and policy[3] == 0
    assert same
