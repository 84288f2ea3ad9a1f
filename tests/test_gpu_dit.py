"""DiT workload on the GPU: fused attention numerics and streamed == resident."""

from __future__ import annotations

import copy
import math

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # bf16 results vs float32 references


def _attn_ref(q, k, v):
    q, k, v = (t.float().cpu() for t in (q, k, v))
    a = torch.softmax(q @ k.transpose(-1, -2).contiguous() / math.sqrt(q.shape[-1]), -1)
    return a @ v


@pytest.mark.parametrize("sq,sk", [(256, 256), (1000, 64), (2048, 2048)])
def test_fused_attention_matches_float32(gpu, sq, sk):
    gen = torch.Generator(device=gpu).manual_seed(sq + sk)
    q = torch.randn(1, 4, sq, 128, device=gpu, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, 4, sk, 128, device=gpu, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, 4, sk, 128, device=gpu, generator=gen).to(torch.bfloat16)
    got = W.sdpa(q, k, v).float().cpu()
    want = _attn_ref(q, k, v)
    assert float((got - want).norm() / want.norm()) < REL_TOL


def test_dit_streamed_equals_resident(gpu):
    shape = W.DiTShape(n_blocks=5, dim=256, n_heads=2, ffn=688)
    model = W.build_dit(shape, seed=4)
    x, e, ctx = W.dit_inputs(shape, 512, 64, seed=4)
    resident = copy.deepcopy(model).to(gpu)
    with torch.no_grad():
        want = resident(x.to(gpu), e.to(gpu), ctx.to(gpu))
        want32 = copy.deepcopy(model).float()(x.float(), e.float(), ctx.float())
    block = sum(p.numel() * 2 for p in model.blocks[0].parameters())
    mgr = OffloadManager("dit-small")
    mgr.offload(model, OffloadConfig(include_patterns=["blocks.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                                     profiling_iters=1, max_gpu_mem_bytes=4 * block, offload_timing="eager"))
    with torch.no_grad():
        outs = [model(x.to(gpu), e.to(gpu), ctx.to(gpu)) for _ in range(5)]
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed and mgr.plan.resident
    for out in outs:
        assert torch.equal(out, want)
    rel = float((outs[-1].float().cpu() - want32).norm() / want32.norm())
    assert rel < REL_TOL
    rep = mgr.collect_offload_timing()
    assert rep.num_passes >= 2 and 0.0 <= rep.hidden_fraction <= 1.0
    mgr.release()
