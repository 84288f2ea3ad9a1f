"""Shared-memory streaming blocks, the creator/follower protocol and the host copy pool (CPU).

Mirrors the reference's coordinator and session checks
(tests/unit/test_shm_coordinator*.py, test_shared_offload_session.py):
election by atomic creation, readiness, published failures, creator death
by heartbeat expiry, namespace and option validation. Blocks are checked
byte for byte against the packed layout the oracle restates.
"""

from __future__ import annotations

import multiprocessing as mp
import os
import time
import uuid

import numpy as np
import pytest
import torch

from flextensor_amd.allocation_block import AllocationManager, HostPinner
from flextensor_amd.shared_offload import (
    ShmCoordinator,
    ShmCoordinatorError,
    ShmCreatorDiedError,
    ShmCreatorFailedError,
    SharedOffloadSession,
    control_segment_name,
)
from flextensor_amd.shm import SHM_DIR
from oracle import layout as olay


def _ns() -> str:
    return f"fttest_{uuid.uuid4().hex[:10]}"


def _leftovers(ns: str) -> list[str]:
    return [e for e in os.listdir(SHM_DIR) if e.startswith(ns)]


# ---- parallel host copy ---------------------------------------------------------------


@pytest.mark.parametrize("nbytes", [1, 4095, (1 << 20) + 3, (33 << 20) + 17])
@pytest.mark.parametrize("threads", [1, 4])
def test_host_memcpy_bit_exact(nbytes, threads):
    from flextensor_amd import _native as nat

    nat.load()
    piece, old_threads = nat.get_staging_policy()
    nat.set_staging_policy(piece, threads)
    try:
        rng = np.random.default_rng(nbytes + threads)
        src = torch.from_numpy(rng.integers(0, 256, nbytes + 64, dtype=np.uint8))
        dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8)
        nat.host_memcpy(dst.data_ptr() + 32, src.data_ptr() + 7, nbytes)
        assert torch.equal(dst[32:32 + nbytes], src[7:7 + nbytes])
        assert (dst[:32] == 0xA5).all() and (dst[32 + nbytes:] == 0xA5).all()
    finally:
        nat.set_staging_policy(piece, 0)


def test_host_memcpy_rejects_overlap_and_bad_policy():
    from flextensor_amd import _native as nat

    nat.load()
    buf = torch.zeros(4096, dtype=torch.uint8)
    with pytest.raises(nat.FtxError):
        nat.host_memcpy(buf.data_ptr() + 8, buf.data_ptr(), 1024)
    with pytest.raises(nat.FtxError):
        nat.set_staging_policy(1024, 4)  # pieces below 1 MiB
    with pytest.raises(nat.FtxError):
        nat.set_staging_policy(1 << 20, 65)


# ---- shared-memory allocation blocks ----------------------------------------------------


def _tensors(seed=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(7, 33, generator=g).to(torch.bfloat16)
    b = torch.randn(5, 3, generator=g).t()  # Fortran-contiguous: raw storage bytes kept
    c = torch.randint(0, 100, (129,), generator=g, dtype=torch.int32)
    return [a, b, c]


def test_shm_block_creator_packs_and_follower_maps_the_same_bytes():
    ns = _ns()
    name = f"{ns}_b0"
    src = _tensors(1)
    pinner = HostPinner("torch", enabled=False)
    creator = AllocationManager(host_pinner=pinner, pinned_memory=False).block(shm_block_name=name)
    for t in src:
        creator.add(t)
    views = creator.allocate()
    assert creator.is_memory_creator and os.path.exists(os.path.join(SHM_DIR, name))
    offsets, total = olay.packed_layout([t.numel() * t.element_size() for t in src])
    assert creator.tensor_offsets == offsets and creator.nbytes == total
    for t, v in zip(src, views):
        assert torch.equal(t, v) and v.stride() == t.stride()
    # a follower with meta tensors of the same layouts maps the segment and sees the same bytes
    meta = [torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device="meta") for t in src]
    follower = AllocationManager(host_pinner=pinner, pinned_memory=False).block(shm_block_name=name,
                                                                                 load_from_shm=True)
    for t in meta:
        follower.add(t)
    fviews = follower.allocate()
    assert not follower.is_memory_creator
    assert torch.equal(follower.block, creator.block)
    for t, v in zip(src, fviews):
        assert torch.equal(t, v) and v.stride() == t.stride() and v.dtype == t.dtype
    views[0][0, 0] = 7.0  # one mapping, two processes' views of it
    assert float(fviews[0][0, 0]) == 7.0
    del views, fviews
    creator.release()  # the creator removes the name
    assert not os.path.exists(os.path.join(SHM_DIR, name))
    follower.release()
    assert _leftovers(ns) == []


def test_follower_block_smaller_than_its_tensors_is_rejected():
    ns = _ns()
    name = f"{ns}_b0"
    pinner = HostPinner("torch", enabled=False)
    creator = AllocationManager(host_pinner=pinner, pinned_memory=False).block(shm_block_name=name)
    creator.add(torch.zeros(16, dtype=torch.uint8))
    creator.allocate()
    follower = AllocationManager(host_pinner=pinner, pinned_memory=False).block(shm_block_name=name,
                                                                                 load_from_shm=True)
    follower.add(torch.empty(4096, dtype=torch.uint8, device="meta"))
    with pytest.raises(ValueError, match="holds"):
        follower.allocate()
    creator.release()
    assert _leftovers(ns) == []


# ---- coordinator ------------------------------------------------------------------


def test_first_coordinator_is_creator_and_followers_see_ready():
    ns = _ns()
    creator = ShmCoordinator(ns, heartbeat_interval=0.05)
    follower = ShmCoordinator(ns)
    assert creator.is_creator and not follower.is_creator
    with pytest.raises(TimeoutError):
        follower.wait_for_ready(timeout=0.1)
    creator.notify_ready()
    follower.wait_for_ready(timeout=1.0)
    with pytest.raises(RuntimeError, match="only the creator"):
        follower.notify_ready()
    follower.close()
    creator.close()
    assert _leftovers(ns) == []


def test_published_failure_reaches_followers():
    ns = _ns()
    creator = ShmCoordinator(ns)
    follower = ShmCoordinator(ns)
    creator.mark_failed(ValueError("checkpoint is corrupt"))
    with pytest.raises(ShmCreatorFailedError, match="checkpoint is corrupt"):
        follower.wait_for_ready(timeout=1.0)
    follower.close()
    creator.close()


def test_stale_heartbeat_means_creator_died():
    ns = _ns()
    creator = ShmCoordinator(ns, heartbeat_interval=60.0)  # never beats during the test
    follower = ShmCoordinator(ns, keep_alive_seconds=0.2)
    t0 = time.monotonic()
    with pytest.raises(ShmCreatorDiedError) as err:
        follower.wait_for_ready(timeout=5.0)
    assert time.monotonic() - t0 < 3.0
    assert err.value.creator_identity == os.getpid()
    follower.close()
    creator.close()


def test_live_heartbeat_keeps_followers_waiting():
    ns = _ns()
    creator = ShmCoordinator(ns, heartbeat_interval=0.02)
    follower = ShmCoordinator(ns, keep_alive_seconds=0.2)
    with pytest.raises(TimeoutError):
        follower.wait_for_ready(timeout=0.6)  # three keep-alive periods: the creator is still beating
    follower.close()
    creator.close()


def test_profile_round_trip_through_the_namespace():
    from flextensor_amd.profile import TensorManagerState

    ns = _ns()
    state = TensorManagerState(loader_type="allocation_block_transfer", tensor_id_to_name_map={1: "w"},
                               allocation_ordered={}, label_to_size_map={}, block_sizes={}, load_strategy={},
                               release_strategy={}, label_to_block_id={}, stats=[], transfer_to_compute_map={},
                               view_tensors_ids=[], view_tensors_names=[], gpu_tensors_names=["w"],
                               shm_block_name_map={"layers.0": f"{ns}_b0"})
    creator = ShmCoordinator(ns)
    creator.write_profile(state)
    follower = ShmCoordinator(ns)
    got = follower.read_profile()
    assert got.to_dict() == state.to_dict()
    follower.close()
    creator.close()
    assert _leftovers(ns) == []


def _elect(ns, start, done, q):
    start.wait(60)
    c = ShmCoordinator(ns, heartbeat_interval=0.05)
    q.put(c.is_creator)
    done.wait(60)  # every process keeps its handle until all have elected
    c.close()


def test_exactly_one_creator_among_racing_processes():
    ns = _ns()
    ctx = mp.get_context("spawn")
    q, start, done = ctx.Queue(), ctx.Event(), ctx.Event()
    procs = [ctx.Process(target=_elect, args=(ns, start, done, q)) for _ in range(4)]
    for p in procs:
        p.start()
    start.set()
    try:
        roles = [q.get(timeout=60) for _ in procs]
    finally:
        done.set()
        for p in procs:
            p.join(60)
    assert sorted(roles) == [False, False, False, True]
    assert _leftovers(ns) == []


def test_protocol_mismatch_is_rejected():
    from flextensor_amd.shm import SharedSegment

    ns = _ns()
    seg = SharedSegment(control_segment_name(ns), 4096, create=True,
                        initializer=lambda buf: buf.__setitem__(slice(0, 8), b"XXXX\x01\x00\x00\x00"))
    with pytest.raises(ShmCoordinatorError, match="protocol"):
        ShmCoordinator(ns)
    seg.close()


# ---- session -----------------------------------------------------------------------


@pytest.mark.parametrize("bad", ["", "a/b", "-lead", "x" * 97, 3])
def test_session_namespace_validation(bad):
    with pytest.raises(ValueError):
        SharedOffloadSession(bad)


@pytest.mark.parametrize("timeout", [-1, float("nan"), float("inf"), True, "soon"])
def test_session_timeout_validation(timeout):
    with pytest.raises(ValueError):
        SharedOffloadSession.validate_options("ok", wait_timeout=timeout)


def test_namespace_for_is_stable_and_per_manager():
    a = SharedOffloadSession("run1")
    b = SharedOffloadSession("run1")
    assert a.namespace_for("default") == b.namespace_for("default")
    assert a.namespace_for("default") != a.namespace_for("other")
    assert a.namespace_for("default") != SharedOffloadSession("run2").namespace_for("default")
    assert a.namespace_for("default").startswith("ft_") and len(a.namespace_for("default")) == 15
    with pytest.raises(ValueError):
        a.namespace_for("bad/name")


def test_session_rejects_unusable_configs(tmp_path):
    from flextensor_amd.config import OffloadConfig

    s = SharedOffloadSession(_ns())
    kw = dict(creator_model_factory=lambda: None, follower_model_factory=lambda: None)
    with pytest.raises(ValueError, match="enabled"):
        s.offload_from_profile(tmp_path, config=OffloadConfig(enabled=False), **kw)
    with pytest.raises(ValueError, match="allocation_block_transfer"):
        s.offload_from_profile(tmp_path, config=OffloadConfig(transfer_mode="raw_block_transfer"), **kw)
    s.close()
    with pytest.raises(RuntimeError, match="closed"):
        s.offload_from_profile(tmp_path, config=OffloadConfig(), **kw)


def test_creator_failure_is_published_and_cleaned_up(tmp_path):
    """A creator whose profile is missing publishes the failure and removes what it made."""
    from flextensor_amd.config import OffloadConfig

    ns = _ns()
    s = SharedOffloadSession(ns)
    inner = s.namespace_for("default")
    with pytest.raises(FileNotFoundError):
        s.offload_from_profile(tmp_path / "missing", config=OffloadConfig(),
                               creator_model_factory=lambda: None, follower_model_factory=lambda: None)
    assert _leftovers(inner) == []
    s.close()


def test_cleanup_namespace_removes_abandoned_segments():
    from flextensor_amd.shm import SharedSegment

    base = _ns()
    ns = SharedOffloadSession(base).namespace_for("default")
    dead = ShmCoordinator(ns, heartbeat_interval=60.0)
    extra = SharedSegment(f"{ns}_b0", 64, create=True)
    dead._stop.set()
    # simulate a creator that died: its names stay behind when the process is gone
    dead.is_creator = False
    extra.creator = False
    time.sleep(0.05)  # the heartbeat written at creation is now older than the keep-alive below
    SharedOffloadSession.cleanup_namespace(base, manager_names=["default"], timeout=0.0, keep_alive_seconds=1e-3)
    assert _leftovers(ns) == []
    dead.close()
    extra.close()


def test_cleanup_namespace_refuses_a_live_creator():
    base = _ns()
    ns = SharedOffloadSession(base).namespace_for("default")
    live = ShmCoordinator(ns, heartbeat_interval=0.02)
    with pytest.raises(ShmCoordinatorError, match="live creator"):
        SharedOffloadSession.cleanup_namespace(base, manager_names=["default"], timeout=0.1)
    live.close()
    assert _leftovers(ns) == []


def _creator_until_killed(ns, ready, started):
    c = ShmCoordinator(ns, heartbeat_interval=0.05)
    if ready:
        c.notify_ready()
    started.set()
    time.sleep(600)  # the test kills this process long before


@pytest.mark.parametrize("ready", [False, True])
def test_killed_creator_is_detected_and_its_namespace_reclaimed(ready):
    """A creator killed by SIGKILL (no rollback, names left behind) is detected by its expired heartbeat,
    both while initializing and after it was ready; new joiners are refused until cleanup removes the
    names, after which the next coordinator is a fresh creator (tests/unit/shm/test_coordinator.py:198-224,
    tests/unit/shm/test_cleanup.py:231-256)."""
    import signal

    # The creator beats every 0.05 s. A keep-alive of 1.5 s lets a loaded host stall the creator's process
    # for over a second before a live creator reads as dead.
    KEEP_ALIVE = 1.5
    base = _ns()
    ns = SharedOffloadSession(base).namespace_for("default")
    ctx = mp.get_context("spawn")
    started = ctx.Event()
    proc = ctx.Process(target=_creator_until_killed, args=(ns, ready, started))
    proc.start()
    try:
        assert started.wait(120), proc.exitcode
        follower = ShmCoordinator(ns, keep_alive_seconds=KEEP_ALIVE)
        assert not follower.is_creator and follower.is_creator_alive()
        if ready:
            follower.wait_for_ready(timeout=5.0)  # live creator: ready at once
        with pytest.raises(ShmCoordinatorError, match="live creator"):
            SharedOffloadSession.cleanup_namespace(base, manager_names=["default"], timeout=0.2,
                                                   keep_alive_seconds=KEEP_ALIVE)
        proc.kill()
        proc.join(30)
        assert proc.exitcode == -signal.SIGKILL
        time.sleep(KEEP_ALIVE + 0.1)  # past the keep-alive: within it a joiner cannot tell a dead creator from a live one
        with pytest.raises(ShmCreatorDiedError) as err:
            follower.wait_for_ready(timeout=10.0)
        assert err.value.creator_identity == proc.pid and err.value.after_ready is ready
        assert not follower.is_creator_alive()
        follower.close()
        assert _leftovers(ns)  # SIGKILL skips the creator's own removal
        for _ in range(2):  # joiners are refused, and joining does not revive the namespace
            joiner = ShmCoordinator(ns, keep_alive_seconds=KEEP_ALIVE)
            assert not joiner.is_creator
            with pytest.raises(ShmCreatorDiedError):
                joiner.wait_for_ready(timeout=10.0)
            joiner.close()
        SharedOffloadSession.cleanup_namespace(base, manager_names=["default"], timeout=5.0, keep_alive_seconds=KEEP_ALIVE)
        assert _leftovers(ns) == []
        fresh = ShmCoordinator(ns)
        assert fresh.is_creator
        fresh.close()
        assert _leftovers(ns) == []
    finally:
        if proc.is_alive():
            proc.kill()
            proc.join(30)
        SharedOffloadSession.cleanup_namespace(base, manager_names=["default"], timeout=0.0, keep_alive_seconds=1e-3)
