"""End-to-end streaming on the GPU.

Parity bar (the reference's own oracle, L0_cuda_graphs/test_cuda_graphs.py:208-233
and L0_offload_validation/offload_validation.py:629-645): the streamed forward
is bitwise equal to the same model run fully resident with the same kernels;
streamed slot bytes equal the packed host bytes; and the bf16 output is within
1e-2 relative error of a float32 CPU forward.
"""

from __future__ import annotations

import copy

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # bf16 outputs vs the float32 forward


def _rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _resident(model, device):
    m = copy.deepcopy(model).to(device)
    return m


def _small_mlp(n_layers=6, hidden=256, inter=704, seed=0):
    return W.build_mlp_stack(n_layers, hidden, inter, seed=seed)


def _stream(model, device, **cfg):
    # no budget: every unit streams
    base = dict(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1)
    base.update(cfg)
    mgr = OffloadManager(name=f"t{id(model)}")
    mgr.offload(model, OffloadConfig(**base))
    return mgr


class _Shifted(torch.nn.Module):
    """An MLP stack whose forward also reads tensors that are neither parameters nor buffers."""

    def __init__(self, stack):
        super().__init__()
        self.stack = stack
        hidden = stack.layers[0].fc1.in_features
        self.gain = torch.linspace(0.5, 1.5, hidden).to(torch.bfloat16)  # a plain attribute
        self.extra = {"shift": [torch.full((hidden,), 0.25, dtype=torch.bfloat16)]}  # inside containers

    def forward(self, x):
        return self.stack(x * self.gain + self.extra["shift"][0])


def test_plain_tensor_attributes_go_to_the_gpu_and_back(gpu):
    """Tensors the model reaches outside its parameters and buffers are placed on the GPU once, keep
    their identity (every alias sees the device copy), count as unmapped bytes, and return to the host
    on release (tensor_processors.py:685-742, tensor_manager.py:2547-2565)."""
    model = _Shifted(_small_mlp())
    gain, shift = model.gain, model.extra["shift"][0]
    gain_host, shift_host = gain.clone(), shift.clone()
    ref = copy.deepcopy(model).to(gpu)  # .to() moves parameters and buffers only
    ref.gain = ref.gain.to(gpu)
    ref.extra["shift"][0] = ref.extra["shift"][0].to(gpu)
    x = W.mlp_input(16, 256, seed=5).to(gpu)
    with torch.no_grad():
        want = ref(x)
    mgr = _stream(model, gpu, include_patterns=["stack.layers.*"])
    assert model.gain is gain and model.extra["shift"][0] is shift
    assert gain.device.type == "cuda" and shift.device.type == "cuda"
    with torch.no_grad():
        outs = [model(x) for _ in range(4)]
    torch.cuda.synchronize()
    assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.streamed
    for out in outs:
        assert torch.equal(out, want)
    plain_bytes = gain.numel() * gain.element_size() + shift.numel() * shift.element_size()
    assert mgr.get_gpu_memory_usage().unmapped_tensors_bytes >= plain_bytes
    mgr.release()
    assert gain.device.type == "cpu" and torch.equal(gain, gain_host)
    assert shift.device.type == "cpu" and torch.equal(shift, shift_host)


@pytest.mark.parametrize("include,exclude,kept", [(["layers.*.weight"], [], {"fc1.weight", "fc2.weight"}),
                                                   (["layers.*"], ["layers.*.fc2"], {"fc1.weight", "fc1.bias"})])
def test_patterns_choose_the_parameters_a_unit_streams(gpu, include, exclude, kept):
    """Only the parameters that the include patterns name and the exclude patterns leave stream with their
    unit; the rest of the unit stays on the GPU (tensor_discovery.py:326-372,647-700)."""
    model = _small_mlp()
    ref = _resident(model, gpu)
    x = W.mlp_input(16, 256, seed=11).to(gpu)
    with torch.no_grad():
        want = ref(x)
    mgr = _stream(model, gpu, include_patterns=include, exclude_patterns=exclude)
    assert [u.label for u in mgr.units] == [f"layers.{i}" for i in range(6)]
    for u in mgr.units:
        assert {n.removeprefix(u.label + ".") for n in u.names} == kept
    streamed = {id(q) for u in mgr.units for q in u.params}
    assert all(p.device.type == "cuda" for p in model.parameters() if id(p) not in streamed)
    with torch.no_grad():
        outs = [model(x) for _ in range(4)]
    torch.cuda.synchronize()
    assert mgr.phase == OffloadPhase.INFERENCE and len(mgr.plan.streamed) == 6
    for out in outs:
        assert torch.equal(out, want)
    mgr.release()


def test_weights_tied_across_units_stay_resident(gpu, caplog):
    """A parameter held by two streamed units would be read from a ring slot that another unit has since
    refilled; it stays on the GPU for good instead, with a warning, as the reference promotes tensors read
    outside their owning layer (tensor_manager.py:226-272). Outputs stay bitwise equal to resident."""
    model = _small_mlp()
    model.layers[4].fc1.weight = model.layers[1].fc1.weight  # tied: one Parameter in two units
    tied = model.layers[1].fc1.weight
    ref = _resident(model, gpu)  # deepcopy keeps the tie
    assert ref.layers[4].fc1.weight is ref.layers[1].fc1.weight
    x = W.mlp_input(16, 256, seed=9).to(gpu)
    with torch.no_grad():
        want = ref(x)
    with caplog.at_level("WARNING", logger="flextensor_amd.manager"):
        mgr = _stream(model, gpu)
    assert "more than one offload unit" in caplog.text and "layers.1.fc1.weight" in caplog.text
    assert tied.device.type == "cuda" and all(tied is not q for u in mgr.units for q in u.params)
    with torch.no_grad():
        outs = [model(x) for _ in range(5)]
    torch.cuda.synchronize()
    assert mgr.phase == OffloadPhase.INFERENCE and len(mgr.plan.streamed) == 6
    for out in outs:
        assert torch.equal(out, want)
    assert mgr.get_gpu_memory_usage().unmapped_tensors_bytes >= tied.numel() * tied.element_size()
    mgr.release()
    assert tied.device.type == "cpu" and torch.equal(tied, ref.layers[1].fc1.weight.cpu())


@pytest.mark.parametrize("copy_engine", ["auto", "sdma", "kernel"])
@pytest.mark.parametrize("transfer_mode", ["allocation_block_transfer", "raw_block_transfer"])
def test_mlp_streamed_equals_resident(gpu, copy_engine, transfer_mode):
    torch.manual_seed(0)
    model = _small_mlp()
    x = W.mlp_input(16, 256, seed=0)
    ref_model = _resident(model, gpu)
    with torch.no_grad():
        want = ref_model(x.to(gpu))
        want32 = copy.deepcopy(model).float()(x.float())
    mgr = _stream(model, gpu, copy_engine=copy_engine, transfer_mode=transfer_mode)
    outs = []
    with torch.no_grad():
        for _ in range(5):  # discovery, profiling, then three streamed passes
            outs.append(model(x.to(gpu)))
    torch.cuda.synchronize()
    assert mgr.phase == OffloadPhase.INFERENCE
    assert mgr.plan is not None and len(mgr.plan.streamed) == 6
    for out in outs:
        assert torch.equal(out, want)
    assert _rel_err(outs[-1], want32) < REL_TOL
    # every parameter now aliases a ring slot on the device
    assert all(p.device.type == "cuda" for p in model.parameters())
    assert mgr.get_gpu_memory_usage().blocks_bytes > 0
    mgr.release()
    for p, q in zip(model.parameters(), ref_model.parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q.cpu())


def test_slot_bytes_equal_host_bytes(gpu):
    model = _small_mlp(4, 128, 320)
    mgr = _stream(model, gpu)
    x = W.mlp_input(4, 128, seed=1).to(gpu)
    with torch.no_grad():
        for _ in range(2):
            model(x)
    ctrl = mgr.controller
    rt = mgr.loader._transfer_runtime
    s = mgr.loader.backend.current_stream()
    for label in ctrl.block_map_cpu:
        rt.begin()
        t = rt.submit(mgr.loader.label_to_block_id[label], lambda label=label: ctrl.schedule_transfer(label))
        rt.wait_ready(t)
        rt.join()
        s.synchronize()
        host = ctrl.block_map_cpu[label].block
        dev = ctrl.gpu_block_view_map[label]
        assert torch.equal(dev.cpu(), host)
    mgr.release()


def test_partial_budget_uses_reordered_loader(gpu):
    model = _small_mlp(8, 256, 704, seed=3)
    x = W.mlp_input(16, 256, seed=3)
    want = _resident(model, gpu)(x.to(gpu)).detach()
    layer = sum(p.numel() * 2 for p in model.layers[0].parameters())
    mgr = _stream(model, gpu, max_gpu_mem_bytes=5 * layer, num_blocks=2)
    with torch.no_grad():
        outs = [model(x.to(gpu)) for _ in range(4)]
    plan = mgr.plan
    assert plan.resident and plan.streamed and plan.reordered
    assert plan.planned_gpu_bytes <= 5 * layer
    for out in outs:
        assert torch.equal(out, want)
    mgr.release()


def test_offload_timing_reports_hidden_fraction(gpu):
    model = _small_mlp(6, 512, 1408, seed=4)
    x = W.mlp_input(64, 512, seed=4).to(gpu)
    mgr = _stream(model, gpu, offload_timing="eager")
    with torch.no_grad():
        for _ in range(6):
            model(x)
    rep = mgr.collect_offload_timing()
    assert rep is not None and rep.num_passes >= 3
    assert rep.total_transfer_sum > 0 and 0.0 <= rep.hidden_fraction <= 1.0
    mgr.release()


def test_llama_small_generate_matches_resident(gpu):
    shape = W.LlamaShape(n_layers=4, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, inter=688, vocab=1000,
                         max_seq=128)
    model = W.build_llama(shape, seed=2)
    prompt = W.prompt_tokens(1, 24, shape.vocab, seed=2).to(gpu)
    ref = _resident(model, gpu)
    ref.init_cache(1, 64, gpu)
    want_tokens, want_logits = W.generate(ref, prompt, 8)
    mgr = _stream(model, gpu, discovery_iters=1, profiling_iters=1)
    model.init_cache(1, 64, gpu)
    got_tokens, got_logits = W.generate(model, prompt, 8)  # discovery + profiling happen inside
    model.init_cache(1, 64, gpu)
    got2_tokens, got2_logits = W.generate(model, prompt, 8)  # fully streamed
    assert mgr.phase == OffloadPhase.INFERENCE
    for a, b in zip(got2_logits, want_logits):
        assert torch.equal(a, b)
    assert torch.equal(got_tokens, want_tokens) and torch.equal(got2_tokens, want_tokens)
    mgr.release()


def test_fp8_llama_batch8_decode_matches_resident(gpu):
    shape = W.LlamaShape(n_layers=4, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=704, vocab=1000,
                         max_seq=128, fp8=True)
    model = W.build_llama(shape, seed=3)
    prompt = W.prompt_tokens(8, 16, shape.vocab, seed=3).to(gpu)
    ref = _resident(model, gpu)
    ref.init_cache(8, 40, gpu)
    want_tokens, want_logits = W.generate(ref, prompt, 6)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    other = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if not n.startswith("layers."))
    other += sum(b.numel() * b.element_size() for b in model.buffers())
    mgr = _stream(model, gpu, max_gpu_mem_bytes=other + int(3.5 * layer))  # 3 streamed + 1 resident
    model.init_cache(8, 40, gpu)
    W.generate(model, prompt, 6)  # discovery + profiling
    model.init_cache(8, 40, gpu)
    got_tokens, got_logits = W.generate(model, prompt, 6)
    assert mgr.plan.streamed and mgr.plan.resident
    assert torch.equal(got_tokens, want_tokens)
    for a, b in zip(got_logits, want_logits):
        assert torch.equal(a, b)
    mgr.release()


@pytest.mark.parametrize("chunk_mib,staged,n_host", [(1, False, 2), (4, False, 2), (1, True, 2), (1, True, 1),
                                                     (4, True, 3)])
def test_chunked_upload_bit_exact(gpu, chunk_mib, staged, n_host):
    from flextensor_amd.hip import checksum
    from flextensor_amd.scatter import upload_tensors
    from oracle import native as onat

    sizes = W.scatter_sizes(300, 4096, 3 << 20, seed=1)
    gen = torch.Generator().manual_seed(1)
    tensors = []
    for i, n in enumerate(sizes):
        t = torch.randint(-32768, 32767, (n // 2,), generator=gen, dtype=torch.int16).view(torch.bfloat16)
        tensors.append(t.view(W.scatter_shape(n, i)))
    tensors.append(torch.arange(12, dtype=torch.float32).reshape(3, 4).t())  # Fortran layout
    tensors.append(torch.arange(20, dtype=torch.float32).reshape(4, 5)[:, ::2])  # gaps -> C-contiguous
    out = upload_tensors(tensors, gpu, chunk_bytes=chunk_mib << 20, staged=staged, n_host=n_host)
    for src, dst in zip(tensors, out):
        assert dst.shape == src.shape and dst.dtype == src.dtype
        # compare bit patterns: random bf16 words include NaNs
        same_width = torch.int16 if src.element_size() == 2 else torch.int32
        assert torch.equal(dst.cpu().view(same_width), src.view(same_width))
    for src, dst in zip(tensors[:-2], out[:-2]):
        assert dst.stride() == src.stride()
        assert checksum(dst.view(-1).view(torch.uint8)) == onat.checksum64(src.contiguous().view(-1).view(torch.uint8))
    assert out[-2].stride() == (1, 4)
    assert out[-1].is_contiguous()


def test_fp8_llama_with_projections_as_units_matches_resident(gpu):
    """fp8 projections that are offload units of their own (attention, gate, up and down) stream through
    their traps: the decoder groups or fuses only projections whose module call would run nothing else, so
    here it calls each streamed module and its weights are loaded before they are read. Greedy tokens and
    every step's logits equal the resident model's, which takes the grouped and fused launches."""
    shape = W.LlamaShape(n_layers=4, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=704, vocab=1000,
                         max_seq=128, fp8=True)
    model = W.build_llama(shape, seed=5)
    prompt = W.prompt_tokens(8, 16, shape.vocab, seed=5).to(gpu)
    ref = _resident(model, gpu)
    ref.init_cache(8, 40, gpu)
    want_tokens, want_logits = W.generate(ref, prompt, 6)
    units = ["layers.*.attn", "layers.*.gate", "layers.*.up", "layers.*.down"]
    unit_bytes = sum(p.numel() * p.element_size() for p in model.layers[0].parameters()) // 4
    other = sum(p.numel() * p.element_size() for p in model.parameters()) - 4 * 4 * unit_bytes
    other += sum(b.numel() * b.element_size() for b in model.buffers())
    mgr = _stream(model, gpu, include_patterns=units, max_gpu_mem_bytes=other + 8 * unit_bytes)
    model.init_cache(8, 40, gpu)
    W.generate(model, prompt, 6)  # discovery + profiling
    model.init_cache(8, 40, gpu)
    got_tokens, got_logits = W.generate(model, prompt, 6)
    streamed = set(mgr.plan.streamed)
    assert streamed and any(x.endswith((".gate", ".up", ".down")) for x in streamed), sorted(streamed)
    assert torch.equal(got_tokens, want_tokens)
    for i, (a, b) in enumerate(zip(got_logits, want_logits)):
        assert torch.equal(a, b), f"step {i}: max |diff| {float((a - b).abs().max()):.3e}"
    mgr.release()
