"""The reference's convenience API on a streamed model (GPU).

``offload_units`` / ``resident_units`` list the units and the rest, ``pause_profiling``
keeps warm-up passes out of the profile and the phase count
(offload_manager.py:3075-3220), and the configuration is fixed once a model
is managed.
"""

from __future__ import annotations

import copy

import pytest
import torch

import flextensor_amd as ft
from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadPhase

pytestmark = pytest.mark.gpu


def test_units_profiling_pause_and_fixed_config(gpu):
    model = W.build_mlp_stack(8, 256, 704, seed=91)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=2, max_gpu_mem_bytes=5 * layer)
    name = "api-test"
    ft.offload(model, cfg, name=name)
    mgr = ft.get_offload_manager(name)
    x = W.mlp_input(16, 256, seed=91).to(gpu)
    with torch.no_grad():
        model(x)  # discovery
        assert mgr.phase == OffloadPhase.PROFILING
        with ft.pause_profiling(name):
            for _ in range(4):  # warm-up passes: not recorded, not counted
                model(x)
        assert mgr.phase == OffloadPhase.PROFILING and not mgr.durations
        model(x)
        assert mgr.phase == OffloadPhase.PROFILING and all(len(v) == 1 for v in mgr.durations.values())
        model(x)  # second recorded profiling pass: streaming starts
        assert mgr.phase == OffloadPhase.INFERENCE
        assert torch.equal(model(x), resident(x))
    units = [label for label, _ in ft.offload_units(name)]
    assert units == [f"layers.{i}" for i in range(8)]  # every offload unit, streamed or kept resident
    assert mgr.plan.streamed and mgr.plan.resident and sorted(mgr.plan.streamed + mgr.plan.resident) == sorted(units)
    assert all(mod is model.get_submodule(label) for label, mod in ft.offload_units(name))
    assert ft.resident_units(name) == ()  # the stack has nothing outside its layers
    with pytest.raises(RuntimeError, match="release"):
        ft.set_config(OffloadConfig(), name=name)
    assert ft.update_offload_timing(name) is True  # timing is off: nothing to store
    ft.release(name)


def test_skip_discovery_streams_after_iters_before_inference(gpu, caplog):
    model = W.build_mlp_stack(8, 256, 704, seed=92)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, skip_discovery=True,
                        profiling_iters=2, max_gpu_mem_bytes=5 * layer, enable_diagnostics=True)
    name = "skip-discovery"
    ft.offload(model, cfg, name=name)
    mgr = ft.get_offload_manager(name)
    assert mgr.skip_discovery_honored and mgr.phase == OffloadPhase.PROFILING
    x = W.mlp_input(16, 256, seed=92).to(gpu)
    with torch.no_grad():
        want = resident(x)
        with caplog.at_level("INFO", logger="flextensor_amd.manager"):
            for _ in range(mgr.iters_before_inference):
                assert torch.equal(model(x), want)
        assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
        assert mgr.order == [f"layers.{i}" for i in range(8)]  # the first profiling pass recorded the order
        for _ in range(2):
            assert torch.equal(model(x), want)
    assert "plan:" in caplog.text and all(f"layers.{i}" in caplog.text for i in range(8))
    assert "loaded during" in caplog.text and "resident" in caplog.text
    ft.release(name)


def test_manager_seam_and_transfer_benchmark(gpu, tmp_path):
    """The calls a serving loop makes around a streamed forward (offload_manager.py:858-864;
    contrib/vllm/v2/offloader.py:393-401), and the state adoption method (:1924-1960)."""
    model = W.build_mlp_stack(6, 256, 704, seed=93)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=4 * layer)
    src = ft.get_offload_manager("seam-src")
    src.offload(model, cfg)
    x = W.mlp_input(8, 256, seed=93).to(gpu)
    with torch.no_grad():
        want = resident(x)
        for _ in range(2):
            model(x)
        assert src.phase == OffloadPhase.INFERENCE and src.plan.streamed
        for _ in range(3):
            src.sync_prev_onload()
            out = model(x)
            src.join_after_forward()
            assert torch.equal(out, want)
    stats = src.benchmark_transfers()
    assert sorted(stats) == sorted(src.memory_transfer_stats) and max(stats) <= layer and all(v > 0 for v in stats.values())
    assert src.get_layer_label_by_idx() == [f"layers.{i}" for i in range(6)] and src.eager_profiling_iters == 1
    state = src.state()
    ft.release("seam-src")

    twin = W.build_mlp_stack(6, 256, 704, seed=93)
    dst = ft.get_offload_manager("seam-dst")
    dst.offload_from_state(twin, state, cfg)
    assert dst.phase == OffloadPhase.INFERENCE and dst.iters_before_inference == 0
    with pytest.raises(RuntimeError, match="already active"):
        dst.offload_from_state(twin, state, cfg)
    with torch.no_grad():
        assert torch.equal(twin(x), want)
    ft.release("seam-dst")


class _Flaky(torch.nn.Module):
    """A unit that raises after its compute when told to."""

    def __init__(self, inner: torch.nn.Module) -> None:
        super().__init__()
        self.inner = inner
        self.fail = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.inner(x)
        if self.fail:
            raise RuntimeError("unit failed")
        return y


def test_a_failing_unit_leaves_every_phase_usable(gpu):
    """A unit that raises still exits its trap (trap_tensor_mode.py:376-397): its tensors go back in
    discovery and profiling, its slot is released in streaming, and the next forward is exact."""
    model = W.build_mlp_stack(6, 256, 704, seed=94)
    resident = copy.deepcopy(model).to(gpu)
    model.layers = torch.nn.ModuleList(_Flaky(layer) for layer in model.layers)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=4 * layer)
    name = "flaky"
    ft.offload(model, cfg, name=name)
    mgr = ft.get_offload_manager(name)
    x = W.mlp_input(8, 256, seed=94).to(gpu)
    with torch.no_grad():
        want = resident(x)
        for phase in (OffloadPhase.DISCOVERY, OffloadPhase.PROFILING, OffloadPhase.INFERENCE):
            assert mgr.phase == phase
            model.layers[3].fail = True
            with pytest.raises(RuntimeError, match="unit failed"):
                model(x)
            model.layers[3].fail = False
            if phase != OffloadPhase.INFERENCE:
                assert all(p.device.type == "cpu" for p in model.layers[3].parameters())  # handed back
                assert mgr.phase == phase  # the failed pass counted for nothing
            assert torch.equal(model(x), want)
        assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
        for _ in range(2):
            assert torch.equal(model(x), want)
    ft.release(name)


def test_state_dict_and_load_state_dict_while_streaming(gpu):
    """A streamed parameter views a ring slot that holds whichever unit came last; its state dict entry
    comes from the host block, and loaded weights land there (and so in every later pass)."""
    model = W.build_mlp_stack(6, 256, 704, seed=95)
    original = {k: v.clone() for k, v in model.state_dict().items()}
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=4 * layer)
    name = "state-dict"
    ft.offload(model, cfg, name=name)
    mgr = ft.get_offload_manager(name)
    x = W.mlp_input(8, 256, seed=95).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
    streamed = {f"{u}.{n}" for u in mgr.plan.streamed for n in ("fc1.weight", "fc1.bias", "fc2.weight", "fc2.bias")}
    sd = model.state_dict()
    assert set(sd) == set(original)
    for k, v in original.items():
        assert torch.equal(sd[k].cpu(), v), k
        assert (sd[k].device.type == "cpu") == (k in streamed), k  # streamed entries come from the host blocks
    assert isinstance(model.state_dict(keep_vars=True)[next(iter(streamed))], torch.nn.Parameter)

    other = W.build_mlp_stack(6, 256, 704, seed=96)
    with torch.no_grad():
        want = copy.deepcopy(other).to(gpu)(x)
        model.load_state_dict(other.state_dict())
        for _ in range(3):
            assert torch.equal(model(x), want)  # every pass streams the loaded weights
    for k, v in other.state_dict().items():
        assert torch.equal(model.state_dict()[k].cpu(), v), k
    # a load into one streamed unit alone: the next pass streams it too
    unit = mgr.plan.streamed[0]
    third = W.build_mlp_stack(6, 256, 704, seed=97)
    mixed = copy.deepcopy(other)
    mixed.get_submodule(unit).load_state_dict(third.get_submodule(unit).state_dict())
    with torch.no_grad():
        want = copy.deepcopy(mixed).to(gpu)(x)
        model.get_submodule(unit).load_state_dict(third.get_submodule(unit).state_dict())
        for _ in range(3):
            assert torch.equal(model(x), want)
    with pytest.raises(RuntimeError, match="assign=True"):
        model.load_state_dict(other.state_dict(), assign=True)
    ft.release(name)


def test_overlapping_parameter_views_are_refused_at_the_plan(gpu):
    """loaders.py:1217-1243: a streamed parameter that overlaps another parameter's bytes is refused when
    streaming would start, before any tensor moves; the model keeps its aliasing and can be released."""
    model = W.build_mlp_stack(4, 256, 704, seed=97)
    first_w = next(p for p in model.layers[0].parameters() if p.dim() == 2)
    owner_name, bias = next((n, p) for n, p in model.layers[1].named_parameters() if p.dim() == 1)
    owner = model.layers[1].get_submodule(owner_name.rpartition(".")[0]) if "." in owner_name else model.layers[1]
    shared = torch.nn.Parameter(first_w.data.view(-1)[: bias.numel()])
    setattr(owner, owner_name.rpartition(".")[2], shared)
    want = [p.detach().clone() for p in model.parameters()]
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=3 * layer)
    name = "overlap-refused"
    ft.offload(model, cfg, name=name)
    x = W.mlp_input(16, 256, seed=97).to(gpu)
    with torch.no_grad(), pytest.raises(ValueError, match="overlapping byte regions"):
        for _ in range(4):
            model(x)
    assert ft.get_offload_manager(name).phase == OffloadPhase.PROFILING
    ft.release(name)
    for p, w in zip(model.parameters(), want):
        assert p.device.type == "cpu" and torch.equal(p.detach(), w)
    assert shared.untyped_storage().data_ptr() == first_w.untyped_storage().data_ptr()


class _WithHead(torch.nn.Module):
    """An MLP stack (the offload units) followed by a head that no unit holds."""

    def __init__(self, seed):
        super().__init__()
        self.stack = W.build_mlp_stack(4, 256, 704, seed=seed)
        self.head = torch.nn.Linear(256, 8, dtype=torch.bfloat16)
        with torch.no_grad():
            self.head.weight.copy_(torch.randn(8, 256, generator=torch.Generator().manual_seed(seed)) * 0.05)

    def forward(self, x):
        return self.head(self.stack(x))


def test_one_manager_offloads_a_second_model_after_release(gpu):
    """Everything a cycle sets up, including placing the tensors outside the units on the GPU, is redone
    for the next model the same manager offloads (tests/unit/test_tensor_manager_lifecycle_gaps.py:140-188)."""
    mgr = ft.OffloadManager("reuse")
    cfg = OffloadConfig(include_patterns=["stack.layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1)
    for seed in (21, 22):
        model = _WithHead(seed)
        ref = copy.deepcopy(model).to(gpu)
        x = W.mlp_input(8, 256, seed=seed).to(gpu)
        with torch.no_grad():
            want = ref(x)
        mgr.offload(model, cfg)
        assert model.head.weight.device.type == "cuda"  # outside every unit: placed for good
        with torch.no_grad():
            outs = [model(x) for _ in range(4)]
        torch.cuda.synchronize()
        assert mgr.phase == OffloadPhase.INFERENCE and len(mgr.plan.streamed) == 4
        assert all(torch.equal(o, want) for o in outs)
        mgr.release()
        assert all(p.device.type == "cpu" for p in model.parameters())


def test_user_forward_hooks_see_the_phase_the_pass_moved_to(gpu):
    """The manager's own forward hook runs first, whenever the user registered theirs
    (tests/unit/test_offload_manager_hooks.py:1440-1481): a user hook on the model sees PROFILING after the
    discovery pass and INFERENCE after the profiling pass."""
    model = W.build_mlp_stack(4, 256, 704, seed=31)
    mgr = ft.OffloadManager("hook-order")
    seen_before, seen_after = [], []
    model.register_forward_hook(lambda *_: seen_before.append(mgr.phase))
    mgr.offload(model, OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                                     profiling_iters=1))
    model.register_forward_hook(lambda *_: seen_after.append(mgr.phase))
    x = W.mlp_input(8, 256, seed=31).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    torch.cuda.synchronize()
    want = [OffloadPhase.PROFILING, OffloadPhase.INFERENCE, OffloadPhase.INFERENCE]
    assert seen_before == want and seen_after == want
    mgr.release()
