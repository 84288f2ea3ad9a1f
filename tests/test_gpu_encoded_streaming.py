"""Streaming with exponent-coded blocks (``OffloadConfig(encode_streamed_blocks=True)``).

Each streamed label's transfer is one decode launch that rebuilds the raw block in its ring slot, so
every forward must stay bitwise equal to the resident model's: eager, under a captured graph, with the
reordered loader of a partial budget, through a decoder's generation, and after ``load_state_dict``
rewrote the host blocks (which re-encodes them in place, so a graph captured before the load decodes
the new weights). A pass that the link measurement finds compute-bound streams its blocks raw, and a
replan switches the encoded transfers off and on with the regime.
"""

from __future__ import annotations

import copy

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase

pytestmark = pytest.mark.gpu


def _offload(model, name, **cfg):
    # No link measurement by default: small models are launch-bound, and a pass measured compute-bound
    # keeps its blocks raw (the last two tests); without a measurement every block that shrinks is encoded.
    base = dict(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1,
                encode_streamed_blocks=True, link_benchmark=False)
    base.update(cfg)
    mgr = OffloadManager(name=name)
    mgr.offload(model, OffloadConfig(**base))
    return mgr


def _capture(model, static_x):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        for _ in range(2):
            model(static_x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s), torch.no_grad():
        out = model(static_x)
    return g, out


@pytest.mark.parametrize("budget_layers", [None, 5])
def test_encoded_mlp_streams_bitwise_eager_and_in_graphs(gpu, budget_layers):
    model = W.build_mlp_stack(8, 256, 704, seed=41)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    mgr = _offload(model, f"enc-mlp-{budget_layers}",
                   max_gpu_mem_bytes=None if budget_layers is None else budget_layers * layer)
    x = W.mlp_input(16, 256, seed=41).to(gpu)
    with torch.no_grad():
        want = resident(x)
        outs = [model(x) for _ in range(5)]
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
    if budget_layers is not None:
        assert mgr.plan.resident and mgr.plan.reordered
    ctl = mgr.controller
    assert set(ctl.encoded) == set(ctl.block_map_cpu)  # every streamed block of N(0, 0.02) weights encodes
    for label in ctl.encoded:
        assert ctl.link_bytes(label) < 0.8 * ctl.transfer_bytes(label)
    for out in outs:
        assert torch.equal(out, want)

    static_x = x.clone()
    g, static_out = _capture(model, static_x)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {i}"
        with torch.no_grad():
            assert torch.equal(model(x), want)  # eager streamed work between replays
        torch.cuda.synchronize()
    del g
    mgr.release()
    for p, q in zip(model.parameters(), resident.parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q.cpu())


def test_encoded_llama_generation_matches_resident(gpu):
    shape = W.LlamaShape(n_layers=4, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, inter=688, vocab=1000,
                         max_seq=128)
    model = W.build_llama(shape, seed=43)
    prompt = W.prompt_tokens(1, 24, shape.vocab, seed=43).to(gpu)
    ref = copy.deepcopy(model).to(gpu)
    ref.init_cache(1, 64, gpu)
    want_tokens, want_logits = W.generate(ref, prompt, 8)
    mgr = _offload(model, "enc-llama")
    model.init_cache(1, 64, gpu)
    W.generate(model, prompt, 8)  # discovery and profiling happen inside
    model.init_cache(1, 64, gpu)
    got_tokens, got_logits = W.generate(model, prompt, 8)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.controller.encoded
    assert torch.equal(got_tokens, want_tokens)
    for a, b in zip(got_logits, want_logits):
        assert torch.equal(a, b)
    mgr.release()


def test_load_state_dict_reencodes_and_captured_graphs_follow(gpu):
    model = W.build_mlp_stack(6, 256, 704, seed=45)
    mgr = _offload(model, "enc-load")
    x = W.mlp_input(8, 256, seed=45).to(gpu)
    with torch.no_grad():
        for _ in range(3):
            model(x)
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.controller.encoded
    static_x = x.clone()
    g, static_out = _capture(model, static_x)

    # new weights of another scale: another exponent table for every block
    other = W.build_mlp_stack(6, 256, 704, seed=46)
    with torch.no_grad():
        for p in other.parameters():
            p.mul_(7.0)
    want = copy.deepcopy(other).to(gpu)
    with torch.no_grad():
        model.load_state_dict(other.state_dict())
        for _ in range(2):
            assert torch.equal(model(x), want(x))
    g.replay()
    torch.cuda.synchronize()
    with torch.no_grad():
        assert torch.equal(static_out, want(static_x))
    del g
    mgr.release()


def _mlp_stack_4096(gpu):
    model = W.build_mlp_stack(8, 4096, 11008, seed=0)
    resident = W.build_mlp_stack(8, 4096, 11008, seed=0).to(gpu)
    small, large = (W.mlp_input(m, 4096, seed=0).to(gpu) for m in (16, 32768))
    with torch.no_grad():
        want = {16: resident(small), 32768: resident(large)}
    del resident
    torch.cuda.empty_cache()
    return model, {16: small, 32768: large}, want


def test_a_pass_profiled_compute_bound_streams_its_blocks_raw(gpu):
    """The 4096 -> 11008 -> 4096 stack at 32768 rows computes for longer than its transfers: the decode's
    16 CUs would cost more than the bytes it saves, so no block is encoded."""
    model, x, want = _mlp_stack_4096(gpu)
    mgr = _offload(model, "enc-compute-bound", link_benchmark=True)
    try:
        with torch.no_grad():
            for _ in range(3):
                got = model(x[32768])
        assert mgr.phase == OffloadPhase.INFERENCE and mgr.link is not None and not mgr.link.link_bound
        assert not mgr.controller.encoded
        assert torch.equal(got, want[32768])
    finally:
        mgr.release(preserve_model=False)
        torch.cuda.empty_cache()


def test_a_replan_switches_encoded_blocks_with_the_regime(gpu):
    """Profiled at 16 rows the stack is link-bound and its blocks are encoded. A replan measured on
    32768-row passes finds it compute-bound and its transfers copy the raw blocks; a replan back at 16
    rows decodes again. Every pass is bitwise equal to the resident forward."""
    model, x, want = _mlp_stack_4096(gpu)
    mgr = _offload(model, "enc-replan", max_gpu_mem_bytes=1_000_000_000, link_benchmark=True)
    try:
        with torch.no_grad():
            for _ in range(3):
                got = model(x[16])
        assert torch.equal(got, want[16])
        ctl = mgr.controller
        assert mgr.link.link_bound and ctl.encoded and ctl.use_encoded
        label = next(iter(ctl.encoded))
        assert ctl.link_bytes(label) < ctl.transfer_bytes(label)
        for rows, encoded in ((32768, False), (16, True)):
            n = mgr.request_strategy_replan()
            with torch.no_grad():
                for _ in range(n):
                    assert torch.equal(model(x[rows]), want[rows])
            assert mgr.link.link_bound == encoded and ctl.use_encoded == encoded
            assert (ctl.link_bytes(label) < ctl.transfer_bytes(label)) == encoded
            with torch.no_grad():
                assert torch.equal(model(x[rows]), want[rows])
    finally:
        mgr.release(preserve_model=False)
        torch.cuda.empty_cache()


@pytest.mark.parametrize("source", ["pageable", "shared_memory"])
def test_encoded_blocks_from_pageable_and_shared_memory_sources(gpu, source):
    """Host blocks that are not page-locked (pinned_memory=False) or live in named shared-memory segments:
    the encoded copy is this process's own pinned arena, and the streamed forward stays bitwise equal."""
    import os
    import uuid

    extra = ({"pinned_memory": False} if source == "pageable"
             else {"shm_enabled": True, "shm_namespace": f"ftenc_{uuid.uuid4().hex[:10]}"})
    model = W.build_mlp_stack(8, 256, 704, seed=47)
    resident = copy.deepcopy(model).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    mgr = _offload(model, f"enc-{source}", max_gpu_mem_bytes=4 * layer, **extra)
    x = W.mlp_input(16, 256, seed=47).to(gpu)
    try:
        with torch.no_grad():
            want = resident(x)
            for _ in range(5):
                assert torch.equal(model(x), want)
        ctl = mgr.controller
        assert mgr.plan.streamed and set(ctl.encoded) == set(ctl.block_map_cpu)
        if source == "pageable":
            assert all(not b.block.is_pinned() for b in ctl.block_map_cpu.values())
        else:
            assert all(os.path.exists(os.path.join("/dev/shm", n)) for n in ctl.shm_block_name_map.values())
    finally:
        mgr.release()


def test_a_load_that_does_not_encode_fails_loudly(gpu):
    """Weights of random bit patterns encode to more than their arena holds: the load raises, and every
    later forward raises too instead of decoding the old encoded blocks."""
    model = W.build_mlp_stack(6, 256, 704, seed=49)
    mgr = _offload(model, "enc-outgrow")
    x = W.mlp_input(8, 256, seed=49).to(gpu)
    try:
        with torch.no_grad():
            for _ in range(3):
                model(x)
        assert mgr.phase == OffloadPhase.INFERENCE and mgr.controller.encoded
        noisy = W.build_mlp_stack(6, 256, 704, seed=50)
        g = torch.Generator().manual_seed(50)
        with torch.no_grad():
            for p in noisy.parameters():
                p.view(torch.int16).copy_(torch.randint(-32768, 32767, p.shape, generator=g, dtype=torch.int16))
        with pytest.raises(ValueError, match="streamed unit block"):
            model.load_state_dict(noisy.state_dict())
        with pytest.raises(RuntimeError, match="encoded blocks no longer hold"), torch.no_grad():
            model(x)
    finally:
        mgr.release()
