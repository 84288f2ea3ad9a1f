"""Saved profiles on the GPU: a plan saved from one model streams another.

A profile saved after discovery and profiling is adopted by a fresh model
of the same architecture; streaming starts on its first forward and the
outputs stay bitwise equal to the resident forward.
"""

from __future__ import annotations

import copy

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase, offload_from_profile, release
from flextensor_amd.profile import load_state

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    base = dict(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1)
    base.update(kw)
    return OffloadConfig(**base)


def _layer_bytes(model):
    return sum(p.numel() * p.element_size() for p in model.layers[0].parameters())


def test_saved_profile_streams_a_fresh_model(gpu, tmp_path):
    model = W.build_mlp_stack(8, 256, 704, seed=5)
    x = W.mlp_input(16, 256, seed=5).to(gpu)
    with torch.no_grad():
        want = copy.deepcopy(model).to(gpu)(x)
    cfg = _cfg(max_gpu_mem_bytes=5 * _layer_bytes(model), profile_storage_dir=str(tmp_path))
    mgr = OffloadManager(name="profile-src")
    mgr.offload(model, cfg)
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(model(x), want)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed and mgr.plan.resident
    path = mgr.save_profile()
    src_plan = mgr.plan
    mgr.release()
    st = load_state(tmp_path)
    assert str(tmp_path) in path and st.loader_type == cfg.transfer_mode

    twin = W.build_mlp_stack(8, 256, 704, seed=5)
    offload_from_profile(twin, None, cfg, name="profile-dst")
    from flextensor_amd.manager import get_offload_manager

    dst = get_offload_manager("profile-dst")
    assert dst.phase == OffloadPhase.INFERENCE  # no discovery or profiling passes
    assert dst.plan.streamed == src_plan.streamed and dst.plan.block_data == src_plan.block_data
    assert dst.plan.reordered == src_plan.reordered
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(twin(x), want)
    release("profile-dst")
    for p, q in zip(twin.parameters(), W.build_mlp_stack(8, 256, 704, seed=5).parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q)


def test_load_profile_switches_a_model_in_discovery(gpu, tmp_path):
    model = W.build_mlp_stack(6, 256, 704, seed=6)
    x = W.mlp_input(8, 256, seed=6).to(gpu)
    with torch.no_grad():
        want = copy.deepcopy(model).to(gpu)(x)
    cfg = _cfg(profile_storage_dir=str(tmp_path))
    src = OffloadManager(name="lp-src")
    src.offload(model, cfg)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    src.save_profile()
    src.release()

    twin = W.build_mlp_stack(6, 256, 704, seed=6)
    mgr = OffloadManager(name="lp-dst")
    mgr.offload(twin, cfg)
    assert mgr.phase == OffloadPhase.DISCOVERY
    mgr.load_profile()  # directory from the config, model from the manager
    assert mgr.phase == OffloadPhase.INFERENCE
    with torch.no_grad():
        for _ in range(2):
            assert torch.equal(twin(x), want)
    with pytest.raises(RuntimeError, match="already streaming"):
        mgr.load_profile()
    mgr.release()


def test_profile_with_other_transfer_mode_rejected(gpu, tmp_path):
    model = W.build_mlp_stack(4, 128, 320, seed=7)
    x = W.mlp_input(4, 128, seed=7).to(gpu)
    src = OffloadManager(name="tm-src")
    src.offload(model, _cfg(transfer_mode="raw_block_transfer"))
    with torch.no_grad():
        for _ in range(3):
            model(x)
    src.save_profile(str(tmp_path))
    src.release()
    twin = W.build_mlp_stack(4, 128, 320, seed=7)
    with pytest.raises(ValueError, match="transfer_mode"):
        OffloadManager(name="tm-dst").offload(twin, _cfg(), state=load_state(tmp_path))
