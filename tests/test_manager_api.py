"""Named-manager registry, thread ownership and the GPU memory report, on the CPU.

Cases of the reference's tests/unit/test_offload_manager_thread_guard.py:17-113
(one thread owns each named manager; a race to create one name has one
winner; the error names both threads) and tests/unit/test_gpu_memory_usage.py
(the report's fields and MB properties; it is only available in INFERENCE).
"""

from __future__ import annotations

import logging
import threading
from unittest import mock

import pytest
import torch

import flextensor_amd.manager as M
from flextensor_amd.config import OffloadConfig


@pytest.fixture
def names():
    made: list[str] = []
    yield made
    for n in made:
        M._MANAGERS.pop(n, None)


def test_same_thread_gets_the_same_manager(names):
    names.append("tg-same")
    assert M.get_offload_manager("tg-same") is M.get_offload_manager("tg-same")


def test_other_thread_is_refused_with_both_thread_ids(names):
    names.append("tg-cross")
    M.get_offload_manager("tg-cross")
    owner = threading.get_ident()
    seen: dict[str, object] = {}

    def use() -> None:
        seen["thread"] = threading.get_ident()
        try:
            M.get_offload_manager("tg-cross")
        except RuntimeError as exc:
            seen["error"] = str(exc)

    t = threading.Thread(target=use)
    t.start()
    t.join()
    msg = seen["error"]
    assert "tg-cross" in msg and "thread" in msg and str(owner) in msg and str(seen["thread"]) in msg


def test_different_names_on_different_threads(names):
    names += ["tg-main", "tg-other"]
    M.get_offload_manager("tg-main")
    out: dict[str, object] = {}
    t = threading.Thread(target=lambda: out.setdefault("mgr", M.get_offload_manager("tg-other")))
    t.start()
    t.join()
    assert isinstance(out["mgr"], M.OffloadManager)


def test_racing_creation_has_one_winner(names):
    names.append("tg-race")
    barrier = threading.Barrier(2)
    wins, losses = [], []

    def race() -> None:
        barrier.wait()
        try:
            M.get_offload_manager("tg-race")
            wins.append(1)
        except RuntimeError:
            losses.append(1)

    threads = [threading.Thread(target=race) for _ in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(wins) == 1 and len(losses) == 1


def test_memory_usage_fields_and_megabytes():
    u = M.GPUMemoryUsage(blocks_bytes=100 * 2**20, unmapped_tensors_bytes=50 * 2**20, total_bytes=150 * 2**20)
    assert (u.blocks_mb, u.unmapped_tensors_mb, u.total_mb) == (100.0, 50.0, 150.0)
    half = M.GPUMemoryUsage(int(1.5 * 2**20), 2**19)
    assert half.total_bytes == 2 * 2**20 and (half.blocks_mb, half.unmapped_tensors_mb, half.total_mb) == (1.5, 0.5, 2.0)
    zero = M.GPUMemoryUsage(0, 0, 0)
    assert (zero.total_bytes, zero.total_mb) == (0, 0.0)


def test_memory_usage_only_in_inference(names):
    names.append("mem-phase")
    mgr = M.get_offload_manager("mem-phase")
    with pytest.raises(RuntimeError, match="Cannot get GPU memory usage in phase not_initialized"):
        mgr.get_gpu_memory_usage()
    for phase in (M.OffloadPhase.DISCOVERY, M.OffloadPhase.PROFILING):
        mgr.phase = phase
        with pytest.raises(RuntimeError, match=f"Cannot get GPU memory usage in phase {phase.value}"):
            M.get_gpu_memory_usage("mem-phase")
    mgr.phase = M.OffloadPhase.INFERENCE
    mgr._resident_bytes = 4096
    usage = mgr.get_gpu_memory_usage()
    assert (usage.blocks_bytes, usage.unmapped_tensors_bytes, usage.total_bytes) == (0, 4096, 4096)
    mgr.phase = M.OffloadPhase.NOT_INITIALIZED


def test_offload_block_needs_an_offloaded_model(names):
    names.append("blk-none")
    with pytest.raises(RuntimeError, match="Call offload"):
        M.offload_block("x", name="blk-none")


# ---- skip_discovery, profile_read_only, inert settings (config.py:133-160, 240-250, 377-402) ------------


class _Stack(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList(torch.nn.Linear(4, 4) for _ in range(3))


@pytest.fixture
def host_offload(names):
    """``offload()`` on the host: no library, no device placement."""
    with mock.patch.object(M.nat, "load", lambda: None), \
            mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", lambda self, ts: 0):
        def run(name, **cfg):
            names.append(name)
            mgr = M.get_offload_manager(name)
            mgr.offload(_Stack(), OffloadConfig(**cfg))
            return mgr
        yield run


def test_skip_discovery_honoured_with_module_units(host_offload):
    mgr = host_offload("skip-yes", include_patterns=["layers.*"], skip_discovery=True, profiling_iters=3)
    assert mgr.skip_discovery_honored is True and mgr.phase == M.OffloadPhase.PROFILING
    assert mgr.iters_before_inference == 3
    with pytest.raises(RuntimeError, match="skip_discovery is True"):
        mgr.offload_block("blk")


def test_skip_discovery_falls_back_without_module_units(host_offload, caplog):
    with caplog.at_level("WARNING"):
        mgr = host_offload("skip-no", include_patterns=[], skip_discovery=True, discovery_iters=2, profiling_iters=3)
    assert mgr.skip_discovery_honored is False and mgr.phase == M.OffloadPhase.DISCOVERY and mgr._manual
    assert "running the discovery passes instead" in caplog.text
    assert mgr.iters_before_inference == 5


@pytest.mark.parametrize("d, p, want", [(1, 10, 11), (2, 0, 2), (0, 4, 4)])
def test_iters_before_inference_counts_the_passes(host_offload, d, p, want):
    mgr = host_offload(f"iters-{d}-{p}", include_patterns=["layers.*"], discovery_iters=d, profiling_iters=p)
    assert mgr.iters_before_inference == want


def test_read_only_profile_refuses_to_save(host_offload, tmp_path):
    mgr = host_offload("ro", include_patterns=["layers.*"], profile_read_only=True)
    with pytest.raises(ValueError, match="profile_read_only is True"):
        mgr.save_profile(str(tmp_path))


def test_inert_settings_warn(host_offload, caplog):
    with caplog.at_level("WARNING"):
        host_offload("inert", include_patterns=["layers.*"], transfer_budget_scale=0.9, enable_instrumentation=True)
    assert "transfer_budget_scale has no effect" in caplog.text and "enable_instrumentation has no effect" in caplog.text


def test_profile_mode_torch_function_refused():
    with pytest.raises(ValueError, match="torch_function"):
        OffloadConfig(profile_mode="torch_function")
    assert OffloadConfig(profile_mode="getter").profile_mode == "getter"


def test_out_of_memory_names_what_was_being_placed(names):
    names.append("oom")

    def no_room(self, tensors):
        raise torch.cuda.OutOfMemoryError("HIP out of memory")

    with mock.patch.object(M.nat, "load", lambda: None), \
            mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", no_room):
        with pytest.raises(torch.cuda.OutOfMemoryError, match="tensors outside the offload units") as info:
            M.get_offload_manager("oom").offload(_Stack(), OffloadConfig(include_patterns=["layers.0"]))
    assert "include_patterns" in str(info.value) and isinstance(info.value.__cause__, torch.cuda.OutOfMemoryError)
    mgr = M.get_offload_manager("oom")  # the failed offload() left the manager reusable
    assert mgr.model is None and mgr.phase == M.OffloadPhase.NOT_INITIALIZED and not mgr._hooks


class _Ident(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.lin = torch.nn.Linear(2, 2)

    def forward(self, x):
        return id(self)


class _Holder(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList(_Ident() for _ in range(2))


class _Loader:
    def __init__(self) -> None:
        self.calls: list[tuple[str, str]] = []

    def enter(self, label):
        self.calls.append(("enter", label))

    def exit(self, label):
        self.calls.append(("exit", label))

    def shutdown(self):
        return None


def test_patched_forward_runs_on_a_copy_of_the_module(names):
    """offload_manager.py:1114-1135: a copied model's patched forward must run the copy, not the original."""
    import copy

    names.append("rebind")
    with mock.patch.object(M.nat, "load", lambda: None), \
            mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", lambda self, ts: 0):
        model = _Holder()
        custom = model.layers[1].forward = lambda x: "instance forward"
        mgr = M.get_offload_manager("rebind")
        mgr.offload(model, OffloadConfig(include_patterns=["layers.*"]))
    mgr.phase, mgr.loader = M.OffloadPhase.INFERENCE, _Loader()
    twin = copy.deepcopy(model)
    assert model.layers[0](1) == id(model.layers[0]) and twin.layers[0](1) == id(twin.layers[0])
    assert model.layers[1](1) == "instance forward"
    assert mgr.loader.calls[:2] == [("enter", "layers.0"), ("exit", "layers.0")]
    mgr.phase, mgr.device = M.OffloadPhase.INFERENCE, torch.device("cpu")
    with mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None):
        mgr.release()
    assert "forward" not in model.layers[0].__dict__  # the class forward again
    assert model.layers[1].forward is custom  # the caller's own forward is put back


def test_budget_is_capped_by_available_memory(caplog):
    """gpu_budget.py:66-113: the fractional budget never exceeds free memory plus the allocator cache
    (plus what the manager already placed); a negative cache counts as none; below 256 MiB available it
    refuses (the reference's tests/unit/test_resolve_gpu_budget.py:14-113 cases)."""
    GiB = 2**30
    mgr = M.OffloadManager("budget")
    mgr.device = torch.device("cuda", 0)
    mgr._resident_bytes = 1 * GiB

    def state(free, total, reserved, allocated):
        return (mock.patch.object(M.torch.cuda, "mem_get_info", lambda d: (free, total)),
                mock.patch.object(M.torch.cuda, "memory_reserved", lambda d: reserved),
                mock.patch.object(M.torch.cuda, "memory_allocated", lambda d: allocated))

    mgr.config = OffloadConfig(max_gpu_mem_fraction=0.5)
    a, b, c = state(200 * GiB, 288 * GiB, 10 * GiB, 6 * GiB)
    with a, b, c:
        assert mgr._budget() == 144 * GiB  # fits: uncapped
    a, b, c = state(100 * GiB, 288 * GiB, 10 * GiB, 6 * GiB)
    with a, b, c, caplog.at_level("WARNING"):
        assert mgr._budget() == (100 + 4 + 1) * GiB
    assert "capping the GPU memory budget" in caplog.text
    mgr.config = OffloadConfig(max_gpu_mem_bytes=8 * GiB)
    with a, b, c:
        assert mgr._budget() == 8 * GiB
    mgr.config = OffloadConfig(max_gpu_mem_fraction=0.9)
    a2, b2, c2 = state(200 * GiB, 288 * GiB, 2 * GiB, 7 * GiB)  # allocated above reserved: no reusable cache
    with a2, b2, c2:
        assert mgr._budget() == (200 + 0 + 1) * GiB
    mgr.config = OffloadConfig()
    assert mgr._budget() is None
    mgr.config = OffloadConfig(max_gpu_mem_fraction=0.9)
    a, b, c = state(100 * 2**20, 288 * GiB, 0, 0)
    with a, b, c, pytest.raises(RuntimeError, match="Insufficient free GPU memory"):
        mgr._budget()


def test_overlapping_views_are_refused_before_anything_moves():
    """loaders.py:1217-1243: distinct tensors viewing overlapping bytes of one storage cannot be packed
    into blocks (they would stop aliasing); disjoint views of one storage are accepted."""
    from flextensor_amd.layout import overlapping_views

    model = torch.nn.Sequential(torch.nn.Linear(8, 8), torch.nn.Linear(8, 8), torch.nn.Linear(8, 8))
    mgr = M.OffloadManager("overlap-check")
    mgr.model = model

    def units():
        return [M._Unit(str(i), model[i], list(model[i].parameters()), [f"{i}.weight", f"{i}.bias"])
                for i in range(3)]

    plan = M.StreamPlan(["0", "1"], ["2"], None, {}, False, None, 0)
    mgr.units = units()
    mgr._validate_source_storage(plan)  # separate storages

    backing = torch.zeros(8 * 8 + 8)
    model[0].weight = torch.nn.Parameter(backing[:64].view(8, 8))
    model[0].bias = torch.nn.Parameter(backing[64:])  # disjoint view of the same storage: fine
    mgr.units = units()
    mgr._validate_source_storage(plan)
    assert overlapping_views([model[0].weight], [model[0].bias]) == []

    model[2].bias = torch.nn.Parameter(backing[60:68])  # resident, but overlaps a streamed weight and bias
    mgr.units = units()
    with pytest.raises(ValueError, match=r"overlapping byte regions \(\[\['0.bias', '0.weight', '2.bias'\]\]\)"):
        mgr._validate_source_storage(plan)
    resident_only = M.StreamPlan(["1"], ["0", "2"], None, {}, False, None, 0)
    mgr._validate_source_storage(resident_only)  # no streamed tensor is involved
    M._MANAGERS.pop("overlap-check", None)


# ---- a streaming build that fails after its controller exists (tensor_manager.py:1585-1596) ----------------


class _PreloadFails:
    """Stands in for a loader whose constructor's preload raises (a refused copy, an exhausted device)."""

    def __init__(self, *args, **kwargs) -> None:
        raise RuntimeError("preload copy refused")


@pytest.mark.parametrize("shm", [False, True])
def test_failed_loader_build_restores_sources_and_aborts_the_controller(host_offload, shm):
    import os
    import uuid

    ns = f"ftx_abort_{uuid.uuid4().hex[:8]}"
    extra = {"shm_enabled": True, "shm_namespace": ns} if shm else {}
    mgr = host_offload(f"abort-{shm}", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1,
                       pinned_memory=False, link_benchmark=False, **extra)
    params = [p for u in mgr.units for p in u.params]
    want = [p.detach().clone() for p in params]
    hooks_before = len(mgr._hooks)
    mgr.device = torch.device("cpu")  # the ring slots live on the CPU, as in the controller tests
    mgr.order = [u.label for u in mgr.units]
    with mock.patch.object(M, "PreallocatedBatchTransferTensorLoader", _PreloadFails), \
            mock.patch.object(M, "PreallocatedBatchTransferTensorLoaderReordered", _PreloadFails), \
            mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None):
        with pytest.raises(RuntimeError, match="preload copy refused"):
            mgr._to_inference()
    assert mgr.controller is None and mgr.loader is None and len(mgr._hooks) == hooks_before
    for p, w in zip(params, want):  # packed, released, bound to slot views, then put back
        assert p.device.type == "cpu" and torch.equal(p, w)
    if shm:
        assert not [f for f in os.listdir("/dev/shm") if f.startswith(ns)]  # no segment outlives the build
    assert mgr.phase != M.OffloadPhase.INFERENCE


def test_a_failed_move_in_discovery_puts_back_the_moved_parameters(host_offload):
    """A unit whose upload runs out of memory part way leaves every parameter on the host, and the next
    pass still finds the host originals."""
    mgr = host_offload("enter-oom", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    u = mgr.units[0]
    want = [p.detach().clone() for p in u.params]
    originals = [p.data_ptr() for p in u.params]
    real_to = torch.Tensor.to
    calls = {"n": 0}

    def flaky_to(self, *args, **kwargs):
        calls["n"] += 1
        if calls["n"] == 2:
            raise torch.cuda.OutOfMemoryError("HIP out of memory")
        return real_to(self, "cpu").clone()  # a distinct tensor stands in for the device copy

    mgr.device = torch.device("cpu")
    with mock.patch.object(torch.Tensor, "to", flaky_to):
        with pytest.raises(torch.cuda.OutOfMemoryError):
            mgr._enter(u.label)
    assert [p.data_ptr() for p in u.params] == originals and not mgr._cpu_data
    assert u.label not in mgr._seen_this_pass
    mgr._enter(u.label)  # the retry moves every parameter and keeps the host originals
    assert [mgr._cpu_data[id(p)].data_ptr() for p in u.params] == originals
    mgr._exit(u.label)
    assert all(torch.equal(p, w) for p, w in zip(u.params, want))


def test_host_register_mode_is_refused_before_anything_moves(names):
    """In-place page-locking is refused in this build: offload() says so before touching the model, and
    the native wrapper never reaches hipHostRegister."""
    from flextensor_amd import _native as nat

    names.append("host-reg")
    model = _Stack()
    want = [p.detach().clone() for p in model.parameters()]
    with pytest.raises(ValueError, match="host_register"):
        M.get_offload_manager("host-reg").offload(model, OffloadConfig(pinned_memory_mode="host_register"))
    assert all(torch.equal(p, w) and p.device.type == "cpu" for p, w in zip(model.parameters(), want))
    assert M.get_offload_manager("host-reg").model is None
    with pytest.raises(nat.FtxError, match="refused in this build") as info:
        nat.arena_register(0, 4096)
    assert info.value.code == nat.FTX_ERR_UNSUPPORTED
    # without pinning the mode has nothing to pin and is accepted
    assert OffloadConfig(pinned_memory=False, pinned_memory_mode="host_register").pinned_memory_mode == "host_register"


# ---- the copy policy follows the measured host link (memory_transfer_benchmark.py:59-129) ----------------


def _untouched_default():
    """The library's process-wide copy policy must never change: a manager's policy travels with its copies."""
    def refuse(*a):
        raise AssertionError("a manager changed the library's process-wide copy policy")

    return mock.patch.object(M.nat, "set_copy_policy", refuse)


def _fake_link(kernel_faster_up_to: int):
    """Curves where the zero-copy kernel beats SDMA by 30% up to ``kernel_faster_up_to`` bytes, then trails."""
    from flextensor_amd import link_model as L

    sizes = L.link_probe_sizes(1 << 28)
    sdma = L.CopyCurve("sdma", {n: 0.01 + n / 50e6 for n in sizes})
    kernel = L.CopyCurve("kernel", {n: (sdma.best_ms[n] / 1.3 if n <= kernel_faster_up_to else sdma.best_ms[n] * 1.02)
                                    for n in sizes})
    km, sm, ns = L.choose_copy_policy(sdma, kernel)
    return L.LinkMeasurement(sdma, kernel, km, sm, ns)


@pytest.mark.parametrize("cut", [0, 1 << 18, 1 << 22])
def test_copy_policy_follows_the_measured_curve(host_offload, cut):
    from flextensor_amd import link_model as L

    mgr = host_offload(f"link-{cut}", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    mgr.order = [u.label for u in mgr.units]
    plan = M.plan_streaming(mgr.units, mgr.order, None, 0, 2, 2)
    link = _fake_link(cut)
    assert link.kernel_max_bytes == cut  # the curve alone decides where the kernel stops paying
    with mock.patch.object(M, "measure_link", lambda sizes, dev: link) as _, _untouched_default():
        mgr._choose_copy_policy(plan, None)
    # no profiled durations: the measured policy as it is, at the library's default kernel grid
    assert mgr.link.native_policy().astuple() == (cut, link.split_min_bytes, 1, 0)
    assert mgr.get_memory_transfer_stats() == link.sdma.best_ms
    mgr.plan = plan
    table = mgr.plan_table()
    assert "copy policy (measured)" in table
    assert ("zero-copy kernel for chunks up to %d bytes" % cut in table) if cut else ("SDMA for every chunk" in table)
    # the policy and the per-tensor transfer times travel with the saved plan
    state = M.state_from_plan(mgr.model, mgr.units, plan, {}, "allocation_block_transfer", mgr.link)
    assert state.copy_policy == link.to_dict()
    interp = L.MemoryTransferInterpolator(link.sdma.best_ms)
    t = state.load_strategy[next(iter(state.load_strategy))][0]
    assert t.load_time_ms == pytest.approx(interp.bytes_to_duration(t.size_bytes))
    from flextensor_amd.profile import TensorManagerState

    back = TensorManagerState.from_dict(state.to_dict())
    assert back.copy_policy == state.copy_policy
    restored = L.LinkMeasurement.from_dict(back.copy_policy)
    assert restored.policy() == link.policy() and restored.source == "profile"


def _profiled(mgr, ms_per_unit):
    mgr.order = [u.label for u in mgr.units]
    mgr.durations = {x: [ms_per_unit] for x in mgr.order}
    return M.plan_streaming(mgr.units, mgr.order, None, 0, 2, 2)


def test_a_link_bound_pass_copies_every_slot_with_the_kernel(host_offload):
    from flextensor_amd import link_model as L

    mgr = host_offload("link-bound", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    link = _fake_link(1 << 20)
    plan = _profiled(mgr, 1e-6)  # the units compute for far less than their copies take
    sizes = [mgr._unit(x).nbytes for x in plan.streamed]
    assert L.is_link_bound(1e-6 * len(mgr.order), link.transfer_ms(sizes))
    with mock.patch.object(M, "measure_link", lambda sizes, dev: link), _untouched_default():
        mgr._choose_copy_policy(plan, None)
    assert mgr.link.native_policy().astuple() == (max(1 << 20, max(sizes)), link.split_min_bytes, 1,
                                                  L.RING_KERNEL_GRID)
    assert mgr.link.link_bound and mgr.link.kernel_grid == L.RING_KERNEL_GRID
    assert mgr.link.sdma is link.sdma  # the measured curve stays the transfer model
    assert "link-bound pass" in mgr.link.describe()
    assert mgr.link.pass_compute_ms == pytest.approx(1e-6 * len(mgr.order))
    assert mgr.link.pass_transfer_ms == pytest.approx(link.transfer_ms(sizes))
    back = L.LinkMeasurement.from_dict(mgr.link.to_dict())
    assert (back.kernel_grid, back.link_bound, back.policy()) == (L.RING_KERNEL_GRID, True, mgr.link.policy())
    assert (back.pass_compute_ms, back.pass_transfer_ms) == (mgr.link.pass_compute_ms, mgr.link.pass_transfer_ms)


def test_a_compute_bound_pass_keeps_the_measured_policy(host_offload):
    mgr = host_offload("compute-bound", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    link = _fake_link(1 << 20)
    plan = _profiled(mgr, 1e6)
    with mock.patch.object(M, "measure_link", lambda sizes, dev: link), _untouched_default():
        mgr._choose_copy_policy(plan, None)
    assert mgr.link.native_policy().astuple() == (1 << 20, link.split_min_bytes, 1, 0) and not mgr.link.link_bound
    assert mgr.link.pass_compute_ms == pytest.approx(1e6 * len(mgr.order))  # recorded either way
    assert "pass compute" in mgr.link.describe()


def test_link_bound_rule():
    from flextensor_amd import link_model as L

    assert L.is_link_bound(10.0, 100.0) and L.is_link_bound(39.9, 100.0)
    assert not L.is_link_bound(40.0, 100.0) and not L.is_link_bound(500.0, 100.0)
    assert not L.is_link_bound(0.0, 0.0)  # nothing streams: nothing to choose
    curve = L.CopyCurve("sdma", {1 << 20: 0.02, 1 << 22: 0.08})
    link = L.LinkMeasurement(curve, L.CopyCurve("kernel"), 0, 2**63 - 1, 1)
    assert link.transfer_ms([1 << 20, 1 << 22]) == pytest.approx(0.10)
    assert link.transfer_ms([1 << 21]) == pytest.approx(0.04)  # log-log between the points


def test_saved_policies_without_a_kernel_grid_read_as_the_default():
    from flextensor_amd import link_model as L

    old = {"kernel_max_bytes": 1 << 20, "split_min_bytes": 2**63 - 1, "n_copy_streams": 1}
    link = L.LinkMeasurement.from_dict(old)
    assert (link.kernel_grid, link.link_bound) == (0, False)
    assert (link.pass_compute_ms, link.pass_transfer_ms) == (None, None)
    for bad in ({"kernel_grid": -1}, {"kernel_grid": 1 << 21}, {"link_bound": "yes"}, {"pass_compute_ms": -1.0}):
        with pytest.raises(ValueError, match="out-of-range"):
            L.LinkMeasurement.from_dict({**old, **bad})


def test_saved_policy_is_reapplied_without_measuring(host_offload):
    mgr = host_offload("link-saved", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    mgr.order = [u.label for u in mgr.units]
    plan = M.plan_streaming(mgr.units, mgr.order, None, 0, 2, 2)
    saved = M.state_from_plan(mgr.model, mgr.units, plan, {}, "allocation_block_transfer", _fake_link(1 << 20))

    def no_measuring(*a):
        raise AssertionError("a restored plan must not measure the link")

    with mock.patch.object(M, "measure_link", no_measuring), _untouched_default():
        mgr._choose_copy_policy(plan, saved)
    assert mgr.link.native_policy().kernel_max_bytes == 1 << 20 and mgr.link.source == "profile"


def test_link_benchmark_off_or_explicit_engine_keeps_the_default(host_offload):
    for name, cfg in (("link-off", {"link_benchmark": False}), ("link-sdma", {"copy_engine": "sdma"})):
        mgr = host_offload(name, include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1, **cfg)
        mgr.order = [u.label for u in mgr.units]
        plan = M.plan_streaming(mgr.units, mgr.order, None, 0, 2, 2)
        with mock.patch.object(M, "measure_link", lambda *a: (_ for _ in ()).throw(AssertionError("measured"))), \
                _untouched_default():
            mgr._choose_copy_policy(plan, None)
        assert mgr.link is None and mgr.get_memory_transfer_stats() is None


def test_invalid_saved_policy_is_refused():
    from flextensor_amd import link_model as L

    with pytest.raises(ValueError, match="copy_policy"):
        L.LinkMeasurement.from_dict({"kernel_max_bytes": 1})
    with pytest.raises(ValueError, match="out-of-range"):
        L.LinkMeasurement.from_dict({"kernel_max_bytes": 0, "split_min_bytes": 0, "n_copy_streams": 99})


def test_a_failed_link_measurement_keeps_the_default_policy(host_offload, caplog):
    """Measuring the link is an optimisation: if it fails, streaming goes on with the library's policy."""
    from flextensor_amd import _native as nat

    mgr = host_offload("link-fails", include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1)
    mgr.order = [u.label for u in mgr.units]
    plan = M.plan_streaming(mgr.units, mgr.order, None, 0, 2, 2)

    def fails(*a):
        raise nat.FtxOutOfMemoryError(nat.FTX_ERR_OOM, "hipHostMalloc failed")

    with mock.patch.object(M, "measure_link", fails), _untouched_default(), \
            mock.patch.object(M.torch.cuda, "empty_cache", lambda: None), \
            caplog.at_level(logging.WARNING, logger="flextensor_amd.manager"):
        mgr._choose_copy_policy(plan, None)
    assert mgr.link is None and mgr.get_memory_transfer_stats() is None
    assert "measuring the host link failed" in caplog.text


def test_named_managers_each_copy_under_their_own_policy(host_offload):
    """Named managers copy independently (offload_manager.py:2817-2850, allocation_block.py:104-106).

    A link-bound manager, a compute-bound one and one with no link measurement
    stream their passes in alternation in one process. Every copy of each
    manager's controller carries that manager's engine and policy, the library's
    process-wide policy is never written, and releasing one manager leaves the
    others' copies as they were.
    """
    import functools

    from flextensor_amd import _native as nat
    from flextensor_amd import allocation_block as AB
    from flextensor_amd import link_model as L
    from tests.fakes import FakeBackend, Recorder

    link = _fake_link(1 << 20)
    cases = {  # name: (config, profiled ms per unit)
        "pair-link": ({}, 1e-6),
        "pair-compute": ({}, 1e6),
        "pair-default": ({"link_benchmark": False, "copy_engine": "sdma"}, 1.0),
    }
    rec = Recorder()
    loaders = {cls: functools.partial(getattr(M, cls), backend=FakeBackend(rec))
               for cls in ("PreallocatedBatchTransferTensorLoader", "PreallocatedBatchTransferTensorLoaderReordered")}
    managers = {}
    with mock.patch.object(M, "measure_link", lambda sizes, dev: link), _untouched_default(), \
            mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None), \
            mock.patch.multiple(M, **loaders):
        for name, (cfg, ms) in cases.items():
            mgr = host_offload(name, include_patterns=["layers.*"], discovery_iters=1, profiling_iters=1,
                               pinned_memory=False, **cfg)
            mgr.device = torch.device("cpu")  # the ring slots live on the CPU, as in the controller tests
            _profiled(mgr, ms)
            mgr._to_inference()
            assert mgr.phase == M.OffloadPhase.INFERENCE and mgr.plan.streamed
            managers[name] = mgr
    want = {
        "pair-link": (nat.COPY_AUTO, managers["pair-link"].link.native_policy().astuple()),
        "pair-compute": (nat.COPY_AUTO, (1 << 20, link.split_min_bytes, 1, 0)),
        "pair-default": (nat.COPY_SDMA, None),
    }
    assert managers["pair-link"].link.link_bound and want["pair-link"][1][3] == L.RING_KERNEL_GRID
    assert not managers["pair-compute"].link.link_bound and managers["pair-default"].link is None
    owner = {id(b): name for name, mgr in managers.items() for b in mgr.controller.block_map_cpu.values()}

    copies: list[tuple[str, int, tuple | None]] = []
    real_copy_to = AB.AllocationBlock.copy_to

    def recording_copy_to(self, gpu_view, non_blocking=True, stream=None, mode=nat.COPY_AUTO, policy=None):
        copies.append((owner[id(self)], mode, None if policy is None else policy.astuple()))
        real_copy_to(self, gpu_view, non_blocking, stream, mode, policy)

    with mock.patch.object(AB.AllocationBlock, "copy_to", recording_copy_to), _untouched_default():
        for _ in range(2):  # alternate whole passes of the three managers
            for mgr in managers.values():
                for label in mgr.order:
                    mgr.loader.enter(label)
                    mgr.loader.exit(label)
        assert {name for name, *_ in copies} == set(managers)
        assert all((mode, pol) == want[name] for name, mode, pol in copies), copies
        # the order of managers in the log alternates: no manager's copies ran under another's policy
        runs = [copies[0][0]] + [b[0] for a, b in zip(copies, copies[1:]) if a[0] != b[0]]
        assert len(runs) >= 2 * len(managers) - 1
        # one manager goes; the others keep copying under their own policies
        for mgr in (managers["pair-link"],):
            mgr.loader.shutdown()
            mgr.controller.shutdown()
        copies.clear()
        for name in ("pair-compute", "pair-default"):
            for label in managers[name].order:
                managers[name].loader.enter(label)
                managers[name].loader.exit(label)
        assert copies and all((mode, pol) == want[name] for name, mode, pol in copies)


# ---- release() when teardown fails (tests/unit/test_tensor_manager_pinned_memory_mode.py:306-420) ----


def _inference_manager(monkeypatch, name, loader, pinner):
    """A manager that holds a small host model as if it were streaming it: no GPU needed."""
    monkeypatch.setattr(M.torch.cuda, "synchronize", lambda *a, **k: None)
    mgr = M.OffloadManager(name)
    mgr.model = torch.nn.Sequential(torch.nn.Linear(4, 4))
    mgr.device = torch.device("cuda", 0)
    mgr.loader, mgr._pinner = loader, pinner
    mgr.phase = M.OffloadPhase.INFERENCE
    return mgr


def _assert_reset(mgr):
    assert mgr.model is None and mgr.loader is None and mgr._pinner is None
    assert mgr.phase == M.OffloadPhase.NOT_INITIALIZED


def test_release_ends_pins_and_reraises_when_the_loader_shutdown_fails(monkeypatch):
    loader, pinner = mock.MagicMock(), mock.MagicMock()
    loader.shutdown.side_effect = RuntimeError("simulated SHM teardown failure")
    mgr = _inference_manager(monkeypatch, "rel-loader", loader, pinner)
    with pytest.raises(RuntimeError, match="simulated SHM teardown failure"):
        mgr.release()
    loader.shutdown.assert_called_once()
    pinner.release_all.assert_called_once()
    _assert_reset(mgr)


def test_release_raises_a_pin_release_failure_when_the_loader_shut_down(monkeypatch):
    pinner = mock.MagicMock()
    pinner.release_all.side_effect = RuntimeError("pin release failed")
    mgr = _inference_manager(monkeypatch, "rel-pins", mock.MagicMock(), pinner)
    with pytest.raises(RuntimeError, match="pin release failed"):
        mgr.release()
    _assert_reset(mgr)


def test_release_keeps_the_loader_error_when_the_pins_fail_too(monkeypatch, caplog):
    loader, pinner = mock.MagicMock(), mock.MagicMock()
    loader.shutdown.side_effect = RuntimeError("ROOT CAUSE: SHM teardown failure")
    pinner.release_all.side_effect = RuntimeError("CLEANUP NOISE")
    mgr = _inference_manager(monkeypatch, "rel-both", loader, pinner)
    with caplog.at_level(logging.ERROR, logger="flextensor_amd.manager"), pytest.raises(RuntimeError, match="ROOT CAUSE"):
        mgr.release()
    errors = [r for r in caplog.records if r.levelno == logging.ERROR]
    assert errors and any("release_all" in r.getMessage() for r in errors)
    assert any(r.exc_info is not None for r in errors)
    _assert_reset(mgr)


def test_release_keeps_the_pins_when_the_transfer_stream_cannot_be_synchronised(monkeypatch):
    from flextensor_amd.transfer import TransferStreamSynchronizationError

    loader, pinner = mock.MagicMock(), mock.MagicMock()
    loader.shutdown.side_effect = TransferStreamSynchronizationError("transfer sync failed")
    mgr = _inference_manager(monkeypatch, "rel-sync", loader, pinner)
    with pytest.raises(RuntimeError, match="transfer sync failed"):
        mgr.release()
    pinner.release_all.assert_not_called()  # a copy may still read the pinned blocks
    _assert_reset(mgr)


def test_release_puts_the_tensors_back_before_the_loader_goes(monkeypatch):
    """A parameter views its host block again before the loader shuts down (tensor_manager.py:2398-2401)."""
    seen = []
    loader = mock.MagicMock()
    mgr = _inference_manager(monkeypatch, "rel-order", loader, None)
    weight = mgr.model[0].weight
    host_view = torch.full_like(weight, 7.0)  # the label's host block view of this parameter
    controller = mock.MagicMock()
    controller.block_map_cpu = {"0": mock.MagicMock(shm_segment=None)}
    controller.label_to_cpu_tensor_id_map = {"0": [id(weight)]}
    mgr.controller = controller
    monkeypatch.setattr(mgr, "_cpu_views", lambda label: [host_view])
    loader.shutdown.side_effect = lambda: seen.append(weight.data_ptr() == host_view.data_ptr())
    mgr.release()
    assert seen == [True] and torch.equal(weight, host_view)
    _assert_reset(mgr)


def test_disabled_offload_hands_the_model_back_untouched():
    """OffloadConfig(enabled=False) is the reference's no-op manager (tests/unit/test_offload_manager_phase.py:620-638):
    the model comes back as it was, its forward runs as before, and nothing needs the GPU library."""
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(8, 8), torch.nn.ReLU(), torch.nn.Linear(8, 2))
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    x = torch.randn(3, 8)
    want = model(x)
    mgr = M.OffloadManager("disabled")
    out = mgr.offload(model, OffloadConfig(enabled=False, include_patterns=["0"]))
    assert out is model and mgr.phase == M.OffloadPhase.NOT_INITIALIZED
    assert torch.equal(model(x), want)
    assert all(torch.equal(p, before[n]) and p.device.type == "cpu" for n, p in model.named_parameters())
    mgr.release()  # nothing to release


def _one_label_state(model, label, streamed):
    from flextensor_amd.planner import LayerStatistics, TensorStatistics
    from flextensor_amd.profile import TensorManagerState

    inventory = [n for n, _ in model.named_parameters()]
    ids = {n: i for i, n in enumerate(inventory)}
    ts = [TensorStatistics(ids[n], n, 64, 0.1) for n in streamed]
    state = TensorManagerState(
        loader_type="allocation_block_transfer", tensor_id_to_name_map={i: n for n, i in ids.items()},
        allocation_ordered={0: [label]}, label_to_size_map={label: 64 * len(ts)}, block_sizes={0: 64 * len(ts)},
        load_strategy={label: ts}, release_strategy={label: ts}, label_to_block_id={label: 0},
        stats=[LayerStatistics(label, ts, 1.0)], transfer_to_compute_map={label: label},
        view_tensors_ids=[ids[n] for n in streamed], view_tensors_names=list(streamed),
        gpu_tensors_names=[n for n in inventory if n not in streamed])
    state.validate_internal()
    return state


def test_a_saved_profile_decides_what_a_unit_streams(names):
    """A profile made with other patterns is authoritative, as the reference adopts a profile's strategy over
    the runtime selection config (tests/unit/test_state_adoption.py:447-474): the unit streams the saved
    tensors of its module and the module's other parameters stay resident. A unit that would stream tensors
    outside its module is refused."""
    names.extend(["profile-patterns", "profile-outside"])
    with mock.patch.object(M.nat, "load", lambda: None), mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.OffloadManager, "_to_inference", lambda self, state=None: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", lambda self, ts: 0), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None):
        model = _Stack()
        mgr = M.get_offload_manager("profile-patterns")
        mgr.offload(model, OffloadConfig(include_patterns=["layers.*"]),
                    state=_one_label_state(model, "layers.0", ["layers.0.weight"]))
        assert [(u.label, u.names, u.module is model.layers[0]) for u in mgr.units] == \
            [("layers.0", ["layers.0.weight"], True)]
        other = _Stack()
        with pytest.raises(ValueError, match=r"not all parameters of the module 'layers.0'"):
            M.get_offload_manager("profile-outside").offload(
                other, OffloadConfig(include_patterns=["layers.*"]),
                state=_one_label_state(other, "layers.0", ["layers.1.weight"]))
