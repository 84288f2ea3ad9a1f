"""Allocation blocks, slot sizing, pin lifetime and controller release semantics on the CPU.

The cases are those of the reference's tests/unit/test_allocation_block.py:14-372,
test_allocation_manager.py:9-294, test_allocation_block_controller_release.py:42-93
and test_raw_block_controller_release.py:35-74, restated against this
package's API. A CPU device stands in for the GPU slots, as in those tests;
pinning is disabled, or its native register calls are recorded.
"""

from __future__ import annotations

import os

import pytest
import torch

from flextensor_amd import _native as nat
from flextensor_amd.allocation_block import AllocationBlock, AllocationManager, HostPinner
from flextensor_amd.controllers import AllocationBlockController, RawBlockController
from flextensor_amd.planner import TensorStatistics

NO_PIN = HostPinner("torch", enabled=False)


def _sources() -> list[torch.Tensor]:
    return [torch.ones(12, dtype=torch.float32), torch.ones(15, dtype=torch.float32) * 2,
            torch.ones(13, dtype=torch.int32) * 3, torch.arange(20, dtype=torch.bfloat16).reshape(4, 5).t()]


@pytest.mark.parametrize("alignment", [0, -1, 1.5, True, "128"])
def test_rejects_invalid_memory_alignment(alignment):
    with pytest.raises(ValueError, match="memory_alignment must be a positive integer"):
        AllocationBlock(device="cpu", host_pinner=NO_PIN, memory_alignment=alignment)


def test_allocate_packs_views_at_aligned_offsets():
    src = _sources()
    block = AllocationBlock(device="cpu", host_pinner=NO_PIN, pinned_memory=False)
    for t in src:
        block.add(t)
    views = block.allocate()
    assert [o % 128 for o in block.tensor_offsets] == [0] * len(src)
    for t, v, off in zip(src, views, block.tensor_offsets):
        assert v.dtype == t.dtype and v.shape == t.shape and v.stride() == t.stride()  # Fortran stays Fortran
        assert torch.equal(v, t)
        assert v.storage_offset() * v.element_size() == off and v.untyped_storage().data_ptr() == block.block.data_ptr()
    block.block.zero_()
    assert not views[0].any()  # the views alias the block


def test_copy_to_a_cpu_slot_and_projected_views():
    src = [torch.randn(10), torch.randint(0, 9, (3, 7), dtype=torch.int16)]
    mgr = AllocationManager(host_pinner=NO_PIN, pinned_memory=False)
    block = mgr.block()
    for t in src:
        block.add(t)
    block.allocate()
    slot = mgr.create_max_block(device="cpu")
    views, prefix = block.project_views(slot)
    block.copy_to(prefix)
    for t, v in zip(src, views):
        assert torch.equal(v, t) and v.untyped_storage().data_ptr() == slot.block.data_ptr()
    small = AllocationBlock(device="cpu", block_size=8, host_pinner=NO_PIN, pinned_memory=False)
    with pytest.raises(ValueError, match="does not fit"):
        block.project_views(small)


def test_max_block_sizes_to_the_largest_committed_block():
    mgr = AllocationManager(host_pinner=NO_PIN, pinned_memory=False)
    for t in (torch.ones(10), torch.ones(20), torch.ones(5, dtype=torch.int32), torch.ones(40)):
        b = mgr.block()
        b.add(t)
        b.allocate()
    # the packed total rounds up to the alignment after each tensor (utils.py:114-127): 80 bytes take 128
    assert [b.nbytes for b in mgr.blocks] == [128, 128, 128, 256]
    assert mgr.create_max_block(device="cpu").nbytes == 256
    empty = AllocationManager(host_pinner=NO_PIN, pinned_memory=False)
    empty.block().add(torch.ones(10))  # never allocated
    assert empty.create_max_block(device="cpu").block.numel() == 0


@pytest.fixture
def recorded_pins(monkeypatch):
    calls = {"register": [], "unregister": []}
    monkeypatch.setattr(nat, "arena_register", lambda ptr, n: calls["register"].append((ptr, n)))
    monkeypatch.setattr(nat, "arena_unregister", lambda ptr: calls["unregister"].append(ptr))
    return calls


def test_block_release_keeps_pins(recorded_pins):
    pinner = HostPinner("host_register")
    block = AllocationBlock(device="cpu", block_size=128, host_pinner=pinner)
    assert len(recorded_pins["register"]) == 1 and pinner.pinned_bytes == 128
    block.release()
    assert recorded_pins["unregister"] == [] and pinner.pinned_bytes == 128  # only release_all unpins
    pinner.release_all()
    assert len(recorded_pins["unregister"]) == 1 and pinner.pinned_bytes == 0


def test_manager_release_keeps_pins(recorded_pins):
    pinner = HostPinner("host_register")
    mgr = AllocationManager(host_pinner=pinner)
    for n in (64, 96, 128):
        b = mgr.block()
        b.add(torch.ones(n, dtype=torch.uint8))
        b.allocate()
    assert len(recorded_pins["register"]) == 3
    mgr.release()
    assert recorded_pins["unregister"] == [] and pinner.pinned_bytes == 3 * 128
    pinner.release_all()
    assert len(recorded_pins["unregister"]) == 3


def _stats(tid: int, n: int) -> list[TensorStatistics]:
    return [TensorStatistics(tid, f"t{tid}", n, 0.0)]


def _alloc_controller(release, **kw):
    label = "model.layers.0"
    tensors = {1: torch.arange(64, dtype=torch.uint8)}
    args = {} if release is None else {"release_tensor_memory": release}
    c = AllocationBlockController({0: [label]}, torch.device("cpu"), tensors, {label: _stats(1, 64)}, {label: 0},
                                  host_pinner=NO_PIN, **args, **kw)
    return c, tensors


def _raw_controller(release):
    label = "model.layers.0"
    tensors = {1: torch.arange(64, dtype=torch.uint8)}
    args = {} if release is None else {"release_tensor_memory": release}
    c = RawBlockController({label: 64}, {0: 64}, torch.device("cpu"), tensors, {label: _stats(1, 64)}, {label: 0},
                           host_pinner=NO_PIN, **args)
    return c, tensors


@pytest.mark.parametrize("build", [_alloc_controller, _raw_controller], ids=["allocation", "raw"])
def test_source_release_semantics(build):
    _, kept = build(False)
    assert torch.equal(kept[1], torch.arange(64, dtype=torch.uint8))
    _, released = build(True)
    assert released[1].numel() == 0
    _, default = build(None)
    assert default[1].numel() == 0  # the inference default frees the sources


@pytest.mark.parametrize("build", [_alloc_controller, _raw_controller], ids=["allocation", "raw"])
def test_release_gpu_blocks_drops_every_slot_reference(build):
    c, _ = build(False)
    assert c.block_map_gpu and c.gpu_block_view_map and c.label_to_tensor_views_map and c.tensor_id_to_view_map
    c.release_gpu_blocks()
    assert c.block_map_gpu == {} and c.gpu_block_view_map == {}
    assert c.label_to_tensor_views_map == {} and c.tensor_id_to_view_map == {}
    assert c.get_gpu_memory_bytes() == 0


def test_schedule_transfer_fills_the_slot_views():
    labels = ["a", "b", "c"]
    tensors = {i: torch.randn(16 + 8 * i) for i in range(3)}
    want = {i: t.clone() for i, t in tensors.items()}
    strategy = {x: _stats(i, tensors[i].numel() * 4) for i, x in enumerate(labels)}
    c = AllocationBlockController({0: ["a", "c"], 1: ["b"]}, torch.device("cpu"), tensors, strategy,
                                  {"a": 0, "b": 1, "c": 0}, host_pinner=NO_PIN)
    views = c.get_tensor_id_to_view_mapping()
    assert c.get_gpu_memory_bytes() == c.block_map_cpu["c"].nbytes + c.block_map_cpu["b"].nbytes
    for i, x in enumerate(labels):
        c.schedule_transfer(x)
        assert torch.equal(views[i], want[i])
    # a and c share slot 0: loading c overwrote a's bytes, as the ring intends
    assert views[0].untyped_storage().data_ptr() == views[2].untyped_storage().data_ptr()


def test_failed_construction_restores_released_sources():
    tensors = {1: torch.arange(64, dtype=torch.uint8), 2: torch.arange(32, dtype=torch.uint8)}
    strategy = {"a": _stats(1, 64), "b": _stats(2, 32)}
    with pytest.raises(ValueError, match="no shared-memory block name"):
        AllocationBlockController({0: ["a", "b"]}, torch.device("cpu"), tensors, strategy, {"a": 0, "b": 0},
                                  host_pinner=NO_PIN, shm_block_name_map={"a": "ftx_unused_name_a"})
    assert torch.equal(tensors[1], torch.arange(64, dtype=torch.uint8))  # packed, released, then restored
    assert torch.equal(tensors[2], torch.arange(32, dtype=torch.uint8))
    assert not os.path.exists("/dev/shm/ftx_unused_name_a")  # the segment made for "a" went with the build


class _FailingPinner(HostPinner):
    """Hands out unpinned blocks and fails the n-th request, as an exhausted pinned pool would."""

    def __init__(self, fail_at: int) -> None:
        super().__init__("torch", enabled=False)
        self.calls, self.fail_at = 0, fail_at

    def new_block(self, nbytes: int) -> torch.Tensor:
        self.calls += 1
        if self.calls == self.fail_at:
            raise nat.FtxOutOfMemoryError(nat.FTX_ERR_OOM, "hipHostMalloc failed")
        return super().new_block(nbytes)


def test_raw_controller_failure_restores_released_sources():
    tensors = {1: torch.arange(64, dtype=torch.uint8), 2: torch.arange(16, dtype=torch.float32).reshape(4, 4).t()}
    want = {k: v.clone() for k, v in tensors.items()}
    strategy = {"a": _stats(1, 64), "b": _stats(2, 64)}
    with pytest.raises(nat.FtxOutOfMemoryError):
        RawBlockController({"a": 64, "b": 64}, {0: 64}, torch.device("cpu"), tensors, strategy, {"a": 0, "b": 0},
                           host_pinner=_FailingPinner(fail_at=2))
    for k in tensors:  # "a" was packed and released before "b" failed
        assert torch.equal(tensors[k], want[k])


def test_release_hands_back_block_views_and_ends_the_pins(recorded_pins):
    """tensor_manager.py:2320-2354 and host_pinning.py:314-344: released parameters view their host block
    (no second copy of the model) and the in-place page locks end with the manager."""
    from unittest import mock

    import flextensor_amd.manager as M

    model = torch.nn.Sequential(torch.nn.Linear(4, 4), torch.nn.Linear(4, 4))
    params = list(model[0].parameters())
    want = [p.detach().clone() for p in params]
    tensors = {id(p): p for p in params}
    strategy = {"0": [TensorStatistics(id(p), f"t{i}", p.numel() * p.element_size(), 0.0)
                      for i, p in enumerate(params)]}
    pinner = HostPinner("host_register")
    ctrl = AllocationBlockController({0: ["0"]}, torch.device("cpu"), tensors, strategy, {"0": 0}, host_pinner=pinner)
    ctrl.commit_construction()
    for tid, view in ctrl.get_tensor_id_to_view_mapping().items():
        tensors[tid].data = view  # the parameters alias their slot, as when streaming
    ctrl.schedule_transfer("0")
    host_block = ctrl.block_map_cpu["0"].block
    mgr = M.OffloadManager("release-views")
    mgr.model, mgr.controller, mgr._pinner, mgr.device = model, ctrl, pinner, torch.device("cpu")
    mgr.units = [M._Unit("0", model[0], params, ["0.weight", "0.bias"])]
    assert len(recorded_pins["register"]) == 1 and recorded_pins["unregister"] == []
    with mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None):
        mgr.release()
    for p, w in zip(params, want):
        assert torch.equal(p, w) and p.untyped_storage().data_ptr() == host_block.data_ptr()
    assert len(recorded_pins["unregister"]) == 1 and pinner.pinned_bytes == 0


def test_shared_memory_block_release_keeps_its_pin(recorded_pins):
    """loaders_pin_fallback / allocation_block tests of the reference: only release_all ends pins,
    also for a block living in a shared-memory segment."""
    import uuid

    pinner = HostPinner("host_register")
    block = AllocationBlock(device="cpu", host_pinner=pinner, shm_block_name=f"ftx_t_{uuid.uuid4().hex[:10]}")
    block.add(torch.arange(100, dtype=torch.int32))
    views = block.allocate()
    assert len(recorded_pins["register"]) == 1
    block.release()
    assert recorded_pins["unregister"] == [] and torch.equal(views[0], torch.arange(100, dtype=torch.int32))
    pinner.release_all()
    assert len(recorded_pins["unregister"]) == 1


@pytest.mark.parametrize("raw", [False, True])
def test_failed_cleanup_keeps_the_primary_error_and_a_retry_handle(monkeypatch, raw):
    """loaders.py:1269-1286: a cleanup that fails never replaces the build's own error; the controller stays
    reachable from it so shutdown() can be retried, and the retry restores the released sources."""
    import flextensor_amd.controllers as C

    tensors = {1: torch.arange(64, dtype=torch.uint8), 2: torch.arange(16, dtype=torch.float32)}
    want = {k: v.clone() for k, v in tensors.items()}
    calls = []
    real_restore = C._Rollback.restore

    def flaky_restore(self):
        calls.append(1)
        if len(calls) == 1:
            raise RuntimeError("restore interrupted")
        real_restore(self)

    monkeypatch.setattr(C._Rollback, "restore", flaky_restore)
    with pytest.raises(nat.FtxOutOfMemoryError) as caught:
        if raw:
            RawBlockController({"a": 64, "b": 64}, {0: 64}, torch.device("cpu"), tensors,
                               {"a": _stats(1, 64), "b": _stats(2, 64)}, {"a": 0, "b": 0},
                               host_pinner=_FailingPinner(fail_at=2))
        else:
            AllocationBlockController({0: ["a"], 1: ["b"]}, torch.device("cpu"), tensors,
                                      {"a": _stats(1, 64), "b": _stats(2, 64)}, {"a": 0, "b": 1},
                                      host_pinner=_FailingPinner(fail_at=2))
    err = caught.value
    assert "hipHostMalloc failed" in str(err)  # the primary error, not the cleanup's
    ctrl = err.__dict__["_flextensor_cleanup_controller"]
    assert str(err.__dict__["_flextensor_cleanup_error"]) == "restore interrupted"
    assert tensors[1].numel() == 0  # "a" was packed and released before "b" failed; not yet restored
    ctrl.shutdown()
    for k in tensors:
        assert torch.equal(tensors[k], want[k])
    assert ctrl.block_map_cpu == {}


def test_abort_construction_keeps_the_callers_error(monkeypatch):
    """abort_construction(primary) after a later setup step failed: the cleanup's own failure is attached
    to the caller's error, never raised in its place (loaders.py:1269-1286)."""
    tensors = {1: torch.arange(64, dtype=torch.uint8)}
    want = tensors[1].clone()
    ctrl = RawBlockController({"a": 64}, {0: 64}, torch.device("cpu"), tensors, {"a": _stats(1, 64)}, {"a": 0},
                              host_pinner=_FailingPinner(fail_at=0))
    assert tensors[1].numel() == 0  # packed and released into the host block
    primary = RuntimeError("loader construction failed")
    real = type(ctrl).shutdown
    failures = iter([RuntimeError("first cleanup attempt failed")])

    def flaky(self):
        err = next(failures, None)
        if err is not None:
            raise err
        real(self)

    monkeypatch.setattr(type(ctrl), "shutdown", flaky)
    ctrl.abort_construction(primary)  # does not raise
    assert primary.__dict__["_flextensor_cleanup_controller"] is ctrl
    assert str(primary.__dict__["_flextensor_cleanup_error"]) == "first cleanup attempt failed"
    ctrl.shutdown()  # the retry
    assert torch.equal(tensors[1], want)


# ---- construction rollback: the reference's cases (test_allocation_block_controller.py:32-489) -----------


@pytest.mark.parametrize("commit", [False, True])
def test_sources_are_released_in_the_build_and_restored_unless_committed(commit):
    """test_allocation_block_controller.py:37-64: the build releases each source once its bytes are in the
    host block; shutdown() before commit_construction() gives them back, after it they stay released."""
    t = torch.arange(6, dtype=torch.float32)
    want = t.clone()
    ctrl = AllocationBlockController({0: ["layer.0"]}, torch.device("cpu"), {1: t}, {"layer.0": _stats(1, 24)},
                                     {"layer.0": 0}, host_pinner=NO_PIN)
    assert t.numel() == 0 and t.untyped_storage().nbytes() == 0
    ctrl.schedule_transfer("layer.0", non_blocking=False)
    assert torch.equal(ctrl.get_tensor_id_to_view_mapping()[1], want)
    if commit:
        ctrl.commit_construction()
    ctrl.shutdown()
    if commit:
        assert t.numel() == 0
    else:
        assert torch.equal(t, want)


def _fail_slot_creation(monkeypatch, check):
    def fail(self, device):
        check()
        raise RuntimeError("gpu block creation failed")

    monkeypatch.setattr(AllocationManager, "create_max_block", fail)


@pytest.mark.parametrize("kind", ["private_slice", "external_parameter", "external_view", "expanded_view"])
def test_failed_build_restores_layout_and_surviving_storage(monkeypatch, kind):
    """test_allocation_block_controller.py:442-486: the same tensor object comes back with its offset,
    strides and values; a storage another tensor still holds is viewed again (writes reach the alias), and
    a private storage is not kept alive by the rollback while the build runs."""
    from torch.multiprocessing.reductions import StorageWeakRef

    backing = torch.arange(16.0)
    w = backing[2:5].expand(4, 3) if kind == "expanded_view" else backing[2:14].view(3, 4).t()
    if kind in ("private_slice", "external_parameter"):
        w = torch.nn.Parameter(w, requires_grad=False)
    external = torch.nn.Parameter(backing, requires_grad=False) if kind == "external_parameter" else None
    del backing
    ref = StorageWeakRef(w.untyped_storage())
    want, want_stride, obj = w.clone(), w.stride(), id(w)

    def during_build():
        assert w.numel() == 0
        assert ref.expired() == (kind == "private_slice")

    _fail_slot_creation(monkeypatch, during_build)
    with pytest.raises(RuntimeError, match="gpu block creation failed"):
        AllocationBlockController({0: ["w"]}, torch.device("cpu"), {obj: w, -1: w},  # one tensor, two ids
                                  {"w": _stats(obj, w.numel() * w.element_size())}, {"w": 0}, host_pinner=NO_PIN)
    assert id(w) == obj
    assert w.storage_offset() == 2 and w.stride() == want_stride and torch.equal(w, want)
    if kind != "private_slice":
        assert not ref.expired() and w.untyped_storage().data_ptr() == torch.UntypedStorage._new_with_weak_ptr(
            ref.cdata).data_ptr()
        with torch.no_grad():
            w[0, 0] = 99
        alias = external if external is not None else w._base
        assert alias[2].item() == 99


@pytest.mark.parametrize("keep_backing", [False, True])
def test_failed_build_restores_disjoint_views_of_one_storage_then_retries(monkeypatch, keep_backing):
    """test_allocation_block_controller.py:388-439: two parameters viewing disjoint parts of one storage
    share one storage again after a failed build (the original one while it lives), and a retry builds."""
    from torch.multiprocessing.reductions import StorageWeakRef

    backing = torch.arange(16.0)
    first = torch.nn.Parameter(backing[2:8].reshape(2, 3).t(), requires_grad=False)
    second = torch.nn.Parameter(backing[8:12].view(torch.uint8), requires_grad=False)
    tensors = {1: first, 2: second}
    want = {k: t.clone() for k, t in tensors.items()}
    layout = {k: (t.storage_offset(), t.stride()) for k, t in tensors.items()}
    ref = StorageWeakRef(first.untyped_storage())
    if not keep_backing:
        del backing
    args = ({0: ["left"], 1: ["right"]}, torch.device("cpu"), tensors,
            {"left": _stats(1, 24), "right": _stats(2, 16)}, {"left": 0, "right": 1})
    real = AllocationBlock.project_views

    def fail(self, slot):
        assert first.numel() == second.numel() == 0
        assert ref.expired() is not keep_backing
        raise RuntimeError("view projection failed")

    monkeypatch.setattr(AllocationBlock, "project_views", fail)
    with pytest.raises(RuntimeError, match="view projection failed"):
        AllocationBlockController(*args, host_pinner=NO_PIN)
    assert first.untyped_storage().data_ptr() == second.untyped_storage().data_ptr()
    if keep_backing:
        assert first.untyped_storage().data_ptr() == backing.untyped_storage().data_ptr()
    for k, t in tensors.items():
        assert torch.equal(t, want[k]) and (t.storage_offset(), t.stride()) == layout[k]
    monkeypatch.setattr(AllocationBlock, "project_views", real)
    retry = AllocationBlockController(*args, host_pinner=NO_PIN)
    retry.commit_construction()
    for label in ("left", "right"):
        retry.schedule_transfer(label, non_blocking=False)
    for k, view in retry.get_tensor_id_to_view_mapping().items():
        assert torch.equal(view, want[k])
    retry.shutdown()


@pytest.mark.parametrize("placement", ["same_label", "other_slot", "not_planned"])
@pytest.mark.parametrize("raw", [False, True])
def test_overlapping_sources_are_refused_before_any_is_released(placement, raw):
    """test_allocation_block_controller.py:347-385: distinct tensors with overlapping bytes are refused by the
    controller itself, whether the second one is in the same label, in another slot or in no label at all,
    and every source is left as it was."""
    backing = torch.arange(8.0)
    first = torch.nn.Parameter(backing[:4], requires_grad=False)
    second = torch.nn.Parameter(backing[2:6], requires_grad=False)
    tensors = {1: torch.arange(3.0), 2: first, 3: second}
    want = {k: t.clone() for k, t in tensors.items()}
    ptrs = {k: t.untyped_storage().data_ptr() for k, t in tensors.items()}
    strategy = {"independent": _stats(1, 12), "left": _stats(2, 16)}
    slots, l2b = {0: ["independent", "left"]}, {"independent": 0, "left": 0}
    if placement == "same_label":
        strategy["left"] = strategy["left"] + _stats(3, 16)
    elif placement == "other_slot":
        strategy["right"], slots[1], l2b["right"] = _stats(3, 16), ["right"], 1
    with pytest.raises(ValueError, match="distinct tensor views sharing storage"):
        if raw:
            sizes = {x: 64 for x in strategy}
            RawBlockController(sizes, {b: 64 for b in set(l2b.values())}, torch.device("cpu"), tensors, strategy, l2b,
                               host_pinner=NO_PIN)
        else:
            AllocationBlockController(slots, torch.device("cpu"), tensors, strategy, l2b, host_pinner=NO_PIN)
    assert first.storage_offset() == 0 and second.storage_offset() == 2
    for k, t in tensors.items():
        assert torch.equal(t, want[k]) and t.untyped_storage().data_ptr() == ptrs[k]


def test_one_tensor_under_two_ids_is_not_an_overlap():
    t = torch.arange(8.0)
    ctrl = AllocationBlockController({0: ["a"]}, torch.device("cpu"), {1: t, 2: t}, {"a": _stats(1, 32)}, {"a": 0},
                                     host_pinner=NO_PIN)
    ctrl.schedule_transfer("a", non_blocking=False)
    assert torch.equal(ctrl.get_tensor_id_to_view_mapping()[1], torch.arange(8.0))
    ctrl.shutdown()
