"""Units kept exponent-coded in HBM (``OffloadConfig(encode_resident_blocks=True)``) on the GPU.

The device-side decode (``ftx_expcode_decode_d2d``) rebuilds blocks from device memory bit for bit
against the oracle's encoding, for every size class and escape-heavy data, at the default grid (eight
workgroups per CU) and at a small one; it refuses short or misaligned blocks and writes nothing for a
block of another raw size. A captured decode follows an in-place re-encode. Offloaded models whose
residents do not fit the budget raw keep some encoded, stream fewer units, and stay bitwise equal to
the resident model: eager, in captured graphs, compiled, restored from a saved profile, through
generation, after ``load_state_dict`` and beside encoded streamed blocks; ``release()`` hands the
original weights back.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import OffloadManager, OffloadPhase
from oracle import expcode as oxc
from oracle import expcode_dense as oxd

pytestmark = pytest.mark.gpu


def _bf16_bytes(n: int, seed: int, std: float = 0.02) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n // 2 + 1, generator=g) * std).to(torch.bfloat16).view(torch.uint8).numpy()[:n].copy()


def _dev(a: np.ndarray, gpu, pad: int = 0, fill: int = 0) -> torch.Tensor:
    t = torch.full((a.size + pad,), fill, dtype=torch.uint8, device=gpu)
    t[: a.size].copy_(torch.from_numpy(a))
    return t


def _escape_heavy(n: int, seed: int) -> np.ndarray:
    """bf16 words whose high bytes are random at one word in 40: exponents off every table, in every group."""
    raw = _bf16_bytes(n, seed)
    rng = np.random.default_rng(seed)
    idx = np.arange(1, n, 80)
    raw[idx] = rng.integers(0, 256, idx.size, dtype=np.uint8)
    return raw


@pytest.mark.parametrize("n", [1, 2, 3, 2047, 2048, 2049, 16383, (1 << 20) + 5, 64 << 20])
@pytest.mark.parametrize("kind", ["bf16", "bytes", "mixed"])
@pytest.mark.parametrize("dense", [False, True])
def test_decode_d2d_is_bit_exact(gpu, n, kind, dense):
    from flextensor_amd import expcode

    if kind != "bf16" and n > (1 << 21):
        pytest.skip("escape-heavy data: the smaller sizes cover it")
    print(f"decode_d2d n={n} kind={kind} dense={dense}", flush=True)
    raw = (_bf16_bytes(n, n) if kind == "bf16" else _escape_heavy(n, n) if kind == "mixed"
           else np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8))
    enc = (oxd if dense else oxc).encode(raw)
    src = _dev(enc, gpu, pad=(-enc.size) % 16)
    for grid in (0, 16):
        dst = torch.full((n + 64,), 0xA5, dtype=torch.uint8, device=gpu)
        expcode.decode_d2d(dst, src, n, grid=grid, dense=dense)
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        assert np.array_equal(got[:n], raw), f"grid {grid}"
        assert np.all(got[n:] == 0xA5), f"grid {grid}: wrote past the raw block"


def test_decode_d2d_refusals_and_a_foreign_header(gpu):
    from flextensor_amd import _native as nat
    from flextensor_amd import expcode

    raw = _bf16_bytes(1 << 16, 3)
    enc = oxc.encode(raw)
    src = _dev(enc, gpu, pad=64)
    dst = torch.full((raw.size + 64,), 0x11, dtype=torch.uint8, device=gpu)
    with pytest.raises(nat.FtxError):  # shorter than the planes of its raw size
        nat.call("ftx_expcode_decode_d2d", dst.data_ptr(), src.data_ptr(), 1000, raw.size, 0, None)
    with pytest.raises(nat.FtxError):  # misaligned destination
        nat.call("ftx_expcode_decode_d2d", dst.data_ptr() + 2, src.data_ptr(), src.numel(), raw.size, 0, None)
    with pytest.raises(nat.FtxError):  # misaligned source
        nat.call("ftx_expcode_decode_d2d", dst.data_ptr(), src.data_ptr() + 8, src.numel() - 8, raw.size, 0, None)
    with pytest.raises(ValueError):
        expcode.decode_d2d(dst[:100], src, raw.size)
    # the caller states another raw size than the header's: nothing is written
    expcode.decode_d2d(dst, src, raw.size - 2048)
    torch.cuda.synchronize()
    assert torch.all(dst == 0x11)


def test_dense_decode_refusals_and_a_foreign_header(gpu):
    from flextensor_amd import _native as nat
    from flextensor_amd import expcode

    raw = _escape_heavy(1 << 16, 3)
    enc = oxd.encode(raw)
    src = _dev(enc, gpu, pad=64)
    dst = torch.full((raw.size + 64,), 0x11, dtype=torch.uint8, device=gpu)
    with pytest.raises(nat.FtxError):  # shorter than the sections before Y
        nat.call("ftx_expcode_decode_dense_d2d", dst.data_ptr(), src.data_ptr(), 1000, raw.size, 0, None)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_expcode_decode_dense_d2d", dst.data_ptr() + 2, src.data_ptr(), src.numel(), raw.size, 0, None)
    expcode.decode_d2d(dst, src, raw.size - 2048, dense=True)  # another raw size than the header's
    torch.cuda.synchronize()
    assert torch.all(dst == 0x11)
    # a block cut short inside Y and X: reads stay in the stated bytes, and what they cover decodes
    h = oxd.parse_header(enc)
    assert h["e1"] > 100 and h["e2"] > 10
    short = _dev(enc[: h["off_y"] + 16], gpu)
    expcode.decode_d2d(dst, short, raw.size, dense=True)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dense", [False, True])
def test_device_block_reencodes_in_place_and_captured_decodes_follow(gpu, dense):
    from flextensor_amd import expcode

    fmt = oxd if dense else oxc
    n = (3 << 20) + 2
    a = torch.from_numpy(_bf16_bytes(n, 7))
    b = torch.from_numpy(_bf16_bytes(n, 8, std=3.0))  # another exponent table
    block = expcode.DeviceEncodedBlock.from_raw(a, fmt.encoded_size(b.numpy()) + 4096, gpu, dense=dense)
    assert block.nbytes == fmt.encoded_size(a.numpy()) and block.raw_bytes == n
    assert block.ratio < (0.70 if dense else 0.76)
    assert np.array_equal(block.dev[: block.nbytes].cpu().numpy(), fmt.encode(a.numpy()))
    dst = torch.empty(n, dtype=torch.uint8, device=gpu)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        block.decode(dst)  # warm the launch outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        block.decode(dst)
    for raw in (a, b, a):
        block.reencode(raw)
        for _ in range(2):
            dst.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(dst.cpu(), raw)
    noisy = torch.from_numpy(np.random.default_rng(1).integers(0, 256, n, dtype=np.uint8))
    with pytest.raises(ValueError, match="reserved"):
        block.reencode(noisy)  # escape-heavy: does not fit; the block keeps a
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), a)
    del g


def _layer_bytes(model):
    return sum(p.numel() * p.element_size() for p in model.layers[0].parameters())


def _outside_bytes(model):
    inside = {id(p) for p in model.layers.parameters()}
    return sum(p.numel() * p.element_size() for p in model.parameters() if id(p) not in inside)


def _offload(model, name, budget, **cfg):
    base = dict(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1,
                encode_resident_blocks=True, link_benchmark=False, max_gpu_mem_bytes=budget)
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


@pytest.mark.parametrize("streamed_encoded", [False, True])
def test_mlp_keeps_residents_encoded_and_stays_bitwise(gpu, streamed_encoded):
    """16 layers under a budget of 14: raw, 12 stay resident and 4 stream; encoded, more stay resident
    and fewer stream. Outputs are bitwise those of the resident model, eager and replayed."""
    model = W.build_mlp_stack(16, 512, 1408, seed=51)
    resident = copy.deepcopy(model).to(gpu)
    budget = _outside_bytes(model) + 14 * _layer_bytes(model)
    mgr = _offload(model, f"hbm-mlp-{streamed_encoded}", budget, encode_streamed_blocks=streamed_encoded)
    x = W.mlp_input(8, 512, seed=51).to(gpu)
    try:
        with torch.no_grad():
            want = resident(x)
            outs = [model(x) for _ in range(5)]
        plan = mgr.plan
        assert mgr.phase == OffloadPhase.INFERENCE and plan.encoded_resident
        assert 0 < len(plan.streamed) < 4, plan.streamed
        ctl = mgr.controller
        assert len(ctl.hbm_encoded) == len(plan.encoded_resident)
        assert all(b.ratio < 0.76 for b in ctl.hbm_encoded.values())
        assert bool(ctl.encoded) == streamed_encoded
        usage = mgr.get_gpu_memory_usage()
        assert usage.total_bytes <= budget and plan.planned_gpu_bytes <= budget
        for out in outs:
            assert torch.equal(out, want)
        static_x = x.clone()
        g, static_out = _capture(model, static_x)
        for i in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, want), f"replay {i}"
            with torch.no_grad():
                assert torch.equal(model(x), want)
            torch.cuda.synchronize()
        del g
        assert "exponent-coded in HBM" in mgr.plan_table()
    finally:
        mgr.release()
    for p, q in zip(model.parameters(), resident.parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q.cpu())


def test_llama_generation_with_encoded_residents_matches_resident(gpu):
    shape = W.LlamaShape(n_layers=12, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, inter=688, vocab=1000,
                         max_seq=128)
    model = W.build_llama(shape, seed=53)
    prompt = W.prompt_tokens(1, 24, shape.vocab, seed=53).to(gpu)
    ref = copy.deepcopy(model).to(gpu)
    ref.init_cache(1, 64, gpu)
    want_tokens, want_logits = W.generate(ref, prompt, 8)
    budget = _outside_bytes(model) + 11 * _layer_bytes(model)
    mgr = _offload(model, "hbm-llama", budget)
    try:
        model.init_cache(1, 64, gpu)
        W.generate(model, prompt, 8)  # discovery and profiling happen inside
        model.init_cache(1, 64, gpu)
        got_tokens, got_logits = W.generate(model, prompt, 8)
        assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.encoded_resident and mgr.plan.streamed
        assert torch.equal(got_tokens, want_tokens)
        for a, b in zip(got_logits, want_logits):
            assert torch.equal(a, b)
    finally:
        mgr.release()


def test_load_state_dict_reencodes_hbm_blocks_and_graphs_follow(gpu):
    model = W.build_mlp_stack(16, 512, 1408, seed=55)
    budget = _outside_bytes(model) + 14 * _layer_bytes(model)
    mgr = _offload(model, "hbm-load", budget)
    x = W.mlp_input(8, 512, seed=55).to(gpu)
    try:
        with torch.no_grad():
            for _ in range(3):
                model(x)
        assert mgr.plan.encoded_resident
        static_x = x.clone()
        g, static_out = _capture(model, static_x)
        other = W.build_mlp_stack(16, 512, 1408, seed=56)  # same distribution: fits the reservations
        want = copy.deepcopy(other).to(gpu)
        with torch.no_grad():
            model.load_state_dict(other.state_dict())
            for _ in range(2):
                assert torch.equal(model(x), want(x))
        g.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            assert torch.equal(static_out, want(static_x))
        sd = model.state_dict()
        for k, v in other.state_dict().items():
            assert torch.equal(sd[k].cpu(), v), k
        del g
    finally:
        mgr.release()


def test_a_load_that_outgrows_the_reservation_fails_loudly(gpu):
    """Weights with many more escapes than the reservation holds: the load raises, and every later
    forward raises too instead of computing with the old encoded weights."""
    model = W.build_mlp_stack(16, 512, 1408, seed=57)
    budget = _outside_bytes(model) + 14 * _layer_bytes(model)
    mgr = _offload(model, "hbm-outgrow", budget)
    x = W.mlp_input(8, 512, seed=57).to(gpu)
    try:
        with torch.no_grad():
            for _ in range(3):
                model(x)
        assert mgr.plan.encoded_resident
        noisy = W.build_mlp_stack(16, 512, 1408, seed=58)
        g = torch.Generator().manual_seed(58)
        with torch.no_grad():
            for p in noisy.parameters():  # random bit patterns: most exponents escape
                p.view(torch.int16).copy_(torch.randint(-32768, 32767, p.shape, generator=g, dtype=torch.int16))
        with pytest.raises(ValueError, match="HBM"):
            model.load_state_dict(noisy.state_dict())
        with pytest.raises(RuntimeError, match="HBM"), torch.no_grad():
            model(x)
    finally:
        mgr.release()


def test_compiled_forward_decodes_inside_the_traps(gpu):
    """torch.compile (aot_eager: no code generation) keeps the traps as custom ops; the decode of each unit
    kept in HBM runs inside its trap, and the compiled forward is bitwise the resident one."""
    torch._dynamo.reset()
    model = W.build_mlp_stack(16, 512, 1408, seed=59)
    resident = copy.deepcopy(model).to(gpu)
    budget = _outside_bytes(model) + 14 * _layer_bytes(model)
    mgr = _offload(model, "hbm-compile", budget)
    x = W.mlp_input(8, 512, seed=59).to(gpu)
    try:
        with torch.no_grad():
            for _ in range(3):
                model(x)
            assert mgr.phase == OffloadPhase.INFERENCE and mgr.plan.encoded_resident
            compiled = torch.compile(model, backend="aot_eager", fullgraph=True)
            want = resident(resident(x))
            for _ in range(3):
                assert torch.equal(compiled(compiled(x)), want)
        torch.cuda.synchronize()
    finally:
        torch._dynamo.reset()
        mgr.release()


def test_a_saved_profile_restores_the_units_kept_in_hbm(gpu, tmp_path):
    """A plan saved from a manager that kept units encoded in HBM, restored into a fresh model with the
    option on: the same units stream and the same units are kept encoded, with no discovery or profiling
    pass, and the outputs are bitwise the resident model's."""
    from flextensor_amd.manager import get_offload_manager, offload_from_profile, release

    model = W.build_mlp_stack(16, 512, 1408, seed=61)
    x = W.mlp_input(8, 512, seed=61).to(gpu)
    with torch.no_grad():
        want = copy.deepcopy(model).to(gpu)(x)
    budget = _outside_bytes(model) + 14 * _layer_bytes(model)
    mgr = _offload(model, "hbm-profile-src", budget, profile_storage_dir=str(tmp_path))
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(model(x), want)
    src = mgr.plan
    assert src.encoded_resident
    mgr.save_profile()
    mgr.release()

    twin = W.build_mlp_stack(16, 512, 1408, seed=61)
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1,
                        profiling_iters=1, encode_resident_blocks=True, link_benchmark=False,
                        max_gpu_mem_bytes=budget, profile_storage_dir=str(tmp_path))
    offload_from_profile(twin, None, cfg, name="hbm-profile-dst")
    dst = get_offload_manager("hbm-profile-dst")
    try:
        assert dst.phase == OffloadPhase.INFERENCE
        assert dst.plan.streamed == src.streamed and dst.plan.encoded_resident == src.encoded_resident
        with torch.no_grad():
            for _ in range(3):
                assert torch.equal(twin(x), want)
    finally:
        release("hbm-profile-dst")
    for p, q in zip(twin.parameters(), W.build_mlp_stack(16, 512, 1408, seed=61).parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q)
