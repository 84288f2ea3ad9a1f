"""Streamed forwards captured in a HIP graph and replayed.

Mirrors the reference's CUDA-graph suite (tests/integration/L0_cuda_graphs/
test_cuda_graphs.py:1-30, 208-233): capture during INFERENCE after eager
discovery and profiling; every replay bitwise equal to the eager resident
forward; replays with new static inputs; eager streamed passes between
replays keep working. Each replay is checked, with eager work and
synchronizations in between.
"""

from __future__ import annotations

import copy

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase

pytestmark = pytest.mark.gpu


def _setup(gpu, n_layers, budget_layers, seed, transfer_mode="allocation_block_transfer"):
    model = W.build_mlp_stack(n_layers, 256, 704, seed=seed)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, transfer_mode=transfer_mode,
                        max_gpu_mem_bytes=None if budget_layers is None else budget_layers * layer)
    mgr = OffloadManager(name=f"graph-{seed}-{budget_layers}-{transfer_mode}")
    mgr.offload(model, cfg)
    return model, resident, mgr


def _capture(model, static_x, feedback=2, warmup=3):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        for _ in range(warmup):
            out = static_x
            for _ in range(feedback):
                out = model(out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s), torch.no_grad():
        out = static_x
        for _ in range(feedback):
            out = model(out)
    return g, out


def _resident_feedback(resident, x, feedback=2):
    with torch.no_grad():
        out = x
        for _ in range(feedback):
            out = resident(out)
    return out


@pytest.mark.parametrize("budget_layers,transfer_mode", [(None, "allocation_block_transfer"),
                                                         (None, "raw_block_transfer"),
                                                         (5, "allocation_block_transfer")])
def test_graph_replays_match_resident(gpu, budget_layers, transfer_mode):
    model, resident, mgr = _setup(gpu, 8, budget_layers, seed=21, transfer_mode=transfer_mode)
    x = W.mlp_input(16, 256, seed=21).to(gpu)
    with torch.no_grad():
        for _ in range(3):  # discovery, profiling, first streamed pass (eager)
            model(x)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
    if budget_layers is not None:
        assert mgr.plan.resident and mgr.plan.reordered

    static_x = x.clone()
    g, static_out = _capture(model, static_x)
    want = _resident_feedback(resident, static_x)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {i}"
        with torch.no_grad():  # eager streamed work between replays
            assert torch.equal(_resident_feedback(model, x), _resident_feedback(resident, x))
        torch.cuda.synchronize()

    static_x.copy_(W.mlp_input(16, 256, seed=22).to(gpu))  # new input, same graph
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_out, _resident_feedback(resident, static_x))
    del g
    mgr.release()


def test_capture_before_inference_is_refused(gpu, monkeypatch):
    """The guard fires before any device work, so it is tested without driving a real capture into an error."""
    model, _, mgr = _setup(gpu, 4, None, seed=23)
    x = W.mlp_input(4, 256, seed=23).to(gpu)
    assert mgr.phase == OffloadPhase.DISCOVERY
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="discovery"):
        with torch.no_grad():
            model(x)
    monkeypatch.undo()
    mgr.release()


@pytest.mark.parametrize("budget_layers", [None, 5])
def test_compiled_streamed_forward_matches_resident(gpu, budget_layers):
    """torch.compile (aot_eager: no code generation) keeps the streaming traps as custom ops."""
    torch._dynamo.reset()
    model, resident, mgr = _setup(gpu, 8, budget_layers, seed=31)
    x = W.mlp_input(16, 256, seed=31).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    assert mgr.phase == OffloadPhase.INFERENCE
    compiled = torch.compile(model, backend="aot_eager", fullgraph=True)
    want = _resident_feedback(resident, x)
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(_resident_feedback(compiled, x), want)
    torch.cuda.synchronize()
    torch._dynamo.reset()
    mgr.release()


@pytest.mark.parametrize("budget_layers", [None, 5])
def test_per_unit_compile_fn_matches_resident(gpu, budget_layers):
    """offload(..., compile_fn=...) compiles each unit on its own at INFERENCE (offload_manager.py:2858-2884)."""
    torch._dynamo.reset()
    model = W.build_mlp_stack(8, 256, 704, seed=33)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=None if budget_layers is None else budget_layers * layer)
    compiled_units = []

    def compile_fn(module):
        compiled_units.append(module)
        return torch.compile(module, backend="aot_eager", fullgraph=True)

    mgr = OffloadManager(name=f"compile-fn-{budget_layers}")
    mgr.offload(model, cfg, compile_fn=compile_fn)
    x = W.mlp_input(16, 256, seed=33).to(gpu)
    want = _resident_feedback(resident, x)
    with torch.no_grad():
        model(x)  # discovery runs eagerly: nothing compiled yet
        assert mgr.phase == OffloadPhase.PROFILING and not compiled_units
        model(x)  # profiling, then the switch to streaming compiles the units
        assert mgr.phase == OffloadPhase.INFERENCE
        for _ in range(3):
            assert torch.equal(_resident_feedback(model, x), want)
    units = list(mgr.units)
    assert compiled_units == [u.module for u in units]  # one compiled graph per unit
    assert budget_layers is None or mgr.plan.streamed
    torch.cuda.synchronize()
    mgr.release()
    assert all(u.compiled is None for u in units)
    torch._dynamo.reset()


def test_graph_replay_timing(gpu):
    """offload_timing='cuda_graph': every replay re-times the captured pass (external event nodes)."""
    model = W.build_mlp_stack(6, 512, 1408, seed=41)
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, offload_timing="cuda_graph")
    mgr = OffloadManager(name="graph-timing")
    mgr.offload(model, cfg)
    x = W.mlp_input(64, 512, seed=41).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    mgr.reset_offload_timing()
    g, out = _capture(model, x.clone(), feedback=1, warmup=1)
    mgr.reset_offload_timing()  # drops the eager passes; the captured pass is not a timed pass itself
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        rep = mgr.collect_offload_timing()  # reads the replay that just ran
        assert rep.num_passes == i + 1
        snap = rep.passes[-1]
        assert snap.total_transfer_ms > 0 and snap.total_compute_ms > 0
        assert 0.0 <= rep.hidden_fraction <= 1.0
    del g
    mgr.release()
