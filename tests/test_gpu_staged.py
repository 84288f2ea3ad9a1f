"""GPU parity of the staged copy engine and of streaming from pageable and shared-memory blocks.

Staged copies (pageable source -> pinned staging -> SDMA) must be byte-exact
like every other copy engine; models streamed from pageable or shared-memory
blocks must match the resident forward bitwise, the reference's own oracle
(L0_cuda_graphs/test_cuda_graphs.py:208-233).
"""

from __future__ import annotations

import copy
import os
import subprocess
import sys
import uuid
import warnings

import numpy as np
import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase
from flextensor_amd.shm import SHM_DIR

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def small_pieces(gpu):
    from flextensor_amd import _native as nat

    piece, _ = nat.get_staging_policy()
    nat.set_staging_policy(1 << 20, 4)  # 1 MiB pieces: every copy below crosses several
    yield
    nat.set_staging_policy(piece, 0)


@pytest.mark.parametrize("mode", ["staged", "auto"])
@pytest.mark.parametrize("nbytes", [1, 4095, (1 << 20) + 7, (5 << 20) + 3, 40 << 20])
def test_staged_copy_from_pageable_memory_bit_exact(gpu, small_pieces, mode, nbytes):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    src = torch.from_numpy(np.random.default_rng(nbytes).integers(0, 256, nbytes + 16, dtype=np.uint8))
    keep = src.clone()
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    nat.copy_h2d(dst.data_ptr() + 32, src.data_ptr() + 5, nbytes, nat.COPY_MODES[mode], current_stream(gpu).handle)
    src.fill_(0)  # the source may be reused as soon as the call returns
    torch.cuda.synchronize()
    out = dst.cpu()
    assert torch.equal(out[32:32 + nbytes], keep[5:5 + nbytes])
    assert (out[:32] == 0xA5).all() and (out[32 + nbytes:] == 0xA5).all()


def test_staged_copy_is_refused_while_capturing(gpu):
    from flextensor_amd import _native as nat

    src = torch.zeros(1 << 20, dtype=torch.uint8)
    dst = torch.zeros(1 << 20, dtype=torch.uint8, device=gpu)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    # the refused copy leaves the capture empty, which torch reports as it closes the capture
    with warnings.catch_warnings(), pytest.raises(nat.FtxError) as err:
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty", category=UserWarning)
        with torch.cuda.graph(graph, stream=side):
            nat.copy_h2d(dst.data_ptr(), src.data_ptr(), src.numel(), nat.COPY_STAGED, side.cuda_stream)
    assert err.value.code == nat.FTX_ERR_UNSUPPORTED and "captured" in str(err.value)
    torch.cuda.synchronize()


def _stream_and_compare(gpu, cfg, name, seed=71, budget_layers=4):
    model = W.build_mlp_stack(8, 256, 704, seed=seed)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = cfg.model_copy(update={"max_gpu_mem_bytes": budget_layers * layer})
    mgr = OffloadManager(name=name)
    mgr.offload(model, cfg)
    x = W.mlp_input(16, 256, seed=seed).to(gpu)
    with torch.no_grad():
        want = resident(x)
        for _ in range(5):
            assert torch.equal(model(x), want)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
    return mgr


def test_streaming_from_pageable_blocks_matches_resident(gpu):
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, pinned_memory=False)
    mgr = _stream_and_compare(gpu, cfg, "pageable")
    assert all(not b.block.is_pinned() for b in mgr.controller.block_map_cpu.values())
    mgr.release()


def test_streaming_from_shared_memory_blocks_matches_resident(gpu):
    ns = f"ftgpu_{uuid.uuid4().hex[:10]}"
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, shm_enabled=True, shm_namespace=ns)
    mgr = _stream_and_compare(gpu, cfg, "shm-single")
    names = sorted(mgr.controller.shm_block_name_map.values())
    assert names and all(os.path.exists(os.path.join(SHM_DIR, n)) for n in names)
    st = mgr.state()
    assert st.shm_block_name_map == mgr.controller.shm_block_name_map
    mgr.release()
    assert not any(e.startswith(ns) for e in os.listdir(SHM_DIR))


def test_shared_offload_session_creator_and_follower_match_resident(gpu, tmp_path):
    """Two processes share one host copy: a creator packs the shared blocks, a follower maps them."""
    layers, hidden, inter, seed = 8, 256, 704, 81
    model = W.build_mlp_stack(layers, hidden, inter, seed=seed)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    budget = 4 * layer
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, max_gpu_mem_bytes=budget, profile_storage_dir=str(tmp_path / "prof"))
    mgr = OffloadManager(name="session-profile")
    mgr.offload(model, cfg)
    x = W.mlp_input(16, hidden, seed=seed).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
        want = resident(x).cpu()
    mgr.save_profile()
    mgr.release()
    out = tmp_path / "out"
    out.mkdir()
    ns = f"ftses_{uuid.uuid4().hex[:8]}"
    args = [ns, str(tmp_path / "prof"), str(out)]
    procs = [subprocess.Popen([sys.executable, os.path.join(ROOT, "tests", "shared_worker.py"), *args, str(i), "2",
                               str(layers), str(hidden), str(inter), str(seed), str(budget)],
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True) for i in range(2)]
    logs = []
    for p in procs:
        try:
            logs.append(p.communicate(timeout=300)[0])
        except subprocess.TimeoutExpired:
            p.kill()
            logs.append(p.communicate()[0])
    for p, log in zip(procs, logs):
        assert p.returncode == 0, log[-3000:]
    results = [torch.load(out / f"w{i}.pt", weights_only=True) for i in range(2)]
    roles = sorted(r["info"]["role"] for r in results)
    assert roles == ["creator", "follower"], logs
    for r in results:
        assert r["info"]["streamed"] and r["info"]["shm_blocks"]
        for o in r["outs"]:
            assert torch.equal(o, want)
    assert results[0]["info"]["shm_blocks"] == results[1]["info"]["shm_blocks"]
    from flextensor_amd.shared_offload import SharedOffloadSession

    inner = SharedOffloadSession(ns).namespace_for("default")
    assert all(b.startswith(inner) for b in results[0]["info"]["shm_blocks"])
    assert not any(e.startswith(inner) for e in os.listdir(SHM_DIR))  # nothing left behind
