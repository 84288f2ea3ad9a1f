"""GPU parity of the fp8-weight MFMA linear kernels (``ftx_fp8_linear``): decode (up to 64 rows) and prefill.

The oracle is ``oracle.fp8`` (e4m3fn decoded from the format definition, the
layer in float64). Where every product and partial sum is exact in float32
(small integers times powers of two) the kernel must match the oracle bit for
bit after round-to-nearest-even to bf16; on random data the tolerance is 1e-2
relative error (norm-wise), with a tighter per-element bound.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # bf16 outputs vs the float64 oracle, norm-wise
ELEM_TOL = 2.0 ** -7  # per element, relative to max(|ref|, rms(ref))

# e4m3fn codes of 0, +-1, +-2, +-3, +-4
_SMALL_INT_CODES = np.array([0x00, 0x38, 0xB8, 0x40, 0xC0, 0x44, 0xC4, 0x48, 0xC8], dtype=np.uint8)
_SHAPES = [(1, 16, 16), (8, 1024, 8192), (5, 100, 48), (16, 37, 1040), (17, 300, 528), (33, 96, 160),
           (64, 512, 256), (8, 8192, 4096), (3, 8200, 64)]


@pytest.fixture
def default_config(gpu):
    from flextensor_amd import hip

    hip.set_fp8_linear_config(0, 0)
    yield
    hip.set_fp8_linear_config(0, 0)


def _exact_case(m, n, k, seed):
    rng = np.random.default_rng(seed)
    w_raw = rng.choice(_SMALL_INT_CODES, size=(n, k))
    x = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    scale = rng.choice(np.array([0.25, 0.5, 1.0, 2.0], dtype=np.float32), size=n)
    return x, w_raw, scale


def _to_device(x, w_raw, scale, dev):
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(dev)
    wt = torch.from_numpy(np.ascontiguousarray(w_raw)).view(torch.float8_e4m3fn).to(dev)
    st = torch.from_numpy(np.ascontiguousarray(scale, dtype=np.float32)).to(torch.bfloat16).to(dev)
    return xt, wt, st


def _same_values(got: torch.Tensor, want: torch.Tensor) -> bool:
    """Equal bf16 values (an exact zero may carry either sign)."""
    return torch.equal(got.cpu().float(), want.float())


@pytest.mark.parametrize("m,n,k", _SHAPES)
def test_exact_products_bit_exact(gpu, default_config, m, n, k):
    from flextensor_amd import hip

    x, w_raw, scale = _exact_case(m, n, k, seed=m * 7 + n + k)
    want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16)
    got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu))
    torch.cuda.synchronize()
    assert got.shape == (m, n)
    assert _same_values(got, want)


@pytest.mark.parametrize("waves", [1, 4, 8])
@pytest.mark.parametrize("slice_k", [256, 768, 0])
@pytest.mark.parametrize("m,n,k", [(8, 96, 1040), (40, 64, 4096), (20, 48, 208), (64, 200, 1536), (1, 300, 2560)])
def test_every_launch_shape_bit_exact(gpu, default_config, waves, slice_k, m, n, k):
    from flextensor_amd import hip

    x, w_raw, scale = _exact_case(m, n, k, seed=waves + slice_k + k)
    want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16)
    hip.set_fp8_linear_config(waves, slice_k)
    got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu))
    torch.cuda.synchronize()
    assert _same_values(got, want)


def test_workspace_size_follows_the_split(gpu, default_config):
    from flextensor_amd import hip

    hip.set_fp8_linear_config(0, 1024)
    assert hip.fp8_linear_workspace_bytes(8, 1000, 4096) == 4 * 8 * 1000 * 4
    hip.set_fp8_linear_config(0, 0)
    assert hip.fp8_linear_workspace_bytes(8, 1000, 1024) == 2 * 8 * 1000 * 4  # narrow: slices of two iterations
    assert hip.fp8_linear_workspace_bytes(8, 65536, 1024) == 0  # wide: one slice of four iterations
    hip.set_fp8_linear_config(0, 256)
    assert hip.fp8_linear_workspace_bytes(8, 1000, 512) == 2 * 8 * 1000 * 4
    # the activation slice and eight 16-row weight tiles share 64 KiB of LDS:
    # 8 rows x 4096 bf16 do not fit, so a 4096-wide slice is cut to 1792
    hip.set_fp8_linear_config(0, 4096)
    assert hip.fp8_linear_workspace_bytes(8, 1000, 4096) == 3 * 8 * 1000 * 4


def test_split_calls_in_a_row_stay_exact(gpu, default_config):
    """Split-K calls of different shapes in a row, then the first again: every result stays exact."""
    from flextensor_amd import hip

    hip.set_fp8_linear_config(4, 256)
    cases = [(8, 640, 2048), (3, 70, 1024), (8, 640, 2048), (16, 1024, 512)]
    for m, n, k in cases:
        x, w_raw, scale = _exact_case(m, n, k, seed=n + k)
        want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16)
        for _ in range(3):
            got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu))
            assert _same_values(got, want)


def test_graph_replays_match_eager(gpu, default_config):
    """Captured split-K calls (main kernel + reduce) replay exactly, with eager calls between replays."""
    from flextensor_amd import hip

    x, w_raw, scale = _random_case(8, 4096, 8192, seed=11)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    assert hip.fp8_linear_workspace_bytes(8, 4096, 8192) > 0
    eager = hip.fp8_linear(xt, wt, st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        hip.fp8_linear(xt, wt, st)  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            out = hip.fp8_linear(xt, wt, st)
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        other = hip.fp8_linear(xt, wt, st)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)


@pytest.mark.parametrize("scale_value", [1.0, 0.5])
def test_every_e4m3_code_decodes_exactly(gpu, default_config, scale_value):
    """x = identity rows pick single weights: y[i, j] = w[j, i] * scale for all 256 codes."""
    from flextensor_amd import hip

    codes = np.arange(256, dtype=np.uint8).reshape(16, 16)
    codes[(codes & 0x7F) == 0x7F] = 0x00  # NaN codes would poison the zero products of their row
    w_raw = np.zeros((16, 64), dtype=np.uint8)
    w_raw[:, :16] = codes
    x = np.zeros((16, 64), dtype=np.float32)
    x[np.arange(16), np.arange(16)] = 1.0
    scale = np.full(16, scale_value, dtype=np.float32)
    got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu)).cpu()
    want = torch.from_numpy(ofp8.decode_e4m3fn(codes).T * scale_value).to(torch.bfloat16)
    assert _same_values(got, want)


def _random_case(m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32) * 64.0
    w_raw = torch.from_numpy(np.clip(w, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    scale = (rng.random(n).astype(np.float32) + 0.5) / 448.0
    return x, w_raw, scale


@pytest.mark.parametrize("m,n,k", [(8, 8192, 8192), (8, 1024, 8192), (8, 28672, 8192), (8, 8192, 28672),
                                   (1, 4096, 11008), (64, 256, 4096), (27, 1000, 2000)])
def test_random_matches_float64_oracle(gpu, default_config, m, n, k):
    from flextensor_amd import hip

    x, w_raw, scale = _random_case(m, n, k, seed=m + n + k)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    got = hip.fp8_linear(xt, wt, st).double().cpu()
    # the oracle sees the bf16-rounded activations and scales the kernel sees
    want = torch.from_numpy(ofp8.fp8_linear(xt.float().cpu().numpy(), w_raw, st.float().cpu().numpy()))
    assert float((got - want).norm() / want.norm()) < REL_TOL
    bound = ELEM_TOL * torch.maximum(want.abs(), want.pow(2).mean().sqrt())
    assert bool(((got - want).abs() <= bound).all())


def test_deterministic_and_matches_dequantized_gemm(gpu, default_config):
    from flextensor_amd import workloads as W

    lin = W.Fp8Linear(4096, 2048)
    x, w_raw, scale = _random_case(8, 2048, 4096, seed=5)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    lin.weight.data = wt
    lin.scale.data = st
    with torch.no_grad():
        a = lin(xt.view(8, 1, 4096))
        b = lin(xt.view(8, 1, 4096))
        dequant = torch.nn.functional.linear(xt, wt.to(torch.bfloat16)) * st
    assert a.shape == (8, 1, 2048)
    assert torch.equal(a, b)
    assert float((a.view(8, 2048).double() - dequant.double()).norm() / dequant.double().norm()) < REL_TOL


def test_writes_only_its_output(gpu, default_config):
    """Sentinels around the output stay intact (rows m..15 of the MFMA tile are never stored)."""
    from flextensor_amd import _native as nat

    m, n, k = 5, 40, 64
    x, w_raw, scale = _exact_case(m, n, k, seed=3)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    buf = torch.full((m * n + 256,), 0x5A5A, dtype=torch.int16, device=gpu)
    y = buf[128 : 128 + m * n]
    nat.call("ftx_fp8_linear", xt.data_ptr(), wt.data_ptr(), st.data_ptr(), y.data_ptr(), m, n, k, None, 0,
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = buf.cpu()
    assert (out[:128] == 0x5A5A).all() and (out[128 + m * n :] == 0x5A5A).all()
    want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16).reshape(-1)
    assert _same_values(out[128 : 128 + m * n].view(torch.bfloat16), want)


def test_rejects_bad_arguments(gpu, default_config):
    from flextensor_amd import _native as nat
    from flextensor_amd import hip

    x, w_raw, scale = _exact_case(8, 32, 64, seed=1)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    y = torch.empty(65 * 32, dtype=torch.bfloat16, device=gpu)
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(nat.FtxError) as err:  # an output of more than 2^31 elements
        nat.call("ftx_fp8_linear", xt.data_ptr(), wt.data_ptr(), st.data_ptr(), y.data_ptr(), 1 << 12, 1 << 20, 64,
                 None, 0, s)
    assert err.value.code == nat.FTX_ERR_INVALID
    with pytest.raises(nat.FtxError) as err:  # k not a multiple of 16
        nat.call("ftx_fp8_linear", xt.data_ptr(), wt.data_ptr(), st.data_ptr(), y.data_ptr(), 8, 32, 24, None, 0, s)
    assert err.value.code == nat.FTX_ERR_INVALID
    # weight range past its allocation: a 2 MiB hipMalloc asked to hold 512 x 8192 bytes
    import ctypes

    wbuf = ctypes.c_void_p()
    nat.call("ftx_device_alloc", 1 << 21, ctypes.byref(wbuf))
    try:
        big_x = torch.zeros(8, 8192, dtype=torch.bfloat16, device=gpu)
        big_s = torch.ones(512, dtype=torch.bfloat16, device=gpu)
        big_y = torch.empty(8, 512, dtype=torch.bfloat16, device=gpu)
        with pytest.raises(nat.FtxError) as err:
            nat.call("ftx_fp8_linear", big_x.data_ptr(), wbuf.value, big_s.data_ptr(), big_y.data_ptr(), 8, 512,
                     8192, None, 0, s)
        assert err.value.code == nat.FTX_ERR_INVALID
        assert "weight" in str(err.value)
    finally:
        torch.cuda.synchronize()
        nat.call("ftx_device_free", wbuf.value)
    host_x = torch.zeros(8, 64, dtype=torch.bfloat16)
    with pytest.raises(nat.FtxError) as err:  # host memory as the input
        nat.call("ftx_fp8_linear", host_x.data_ptr(), wt.data_ptr(), st.data_ptr(), y.data_ptr(), 8, 32, 64, None, 0,
                 s)
    assert err.value.code == nat.FTX_ERR_INVALID
    hip.set_fp8_linear_config(0, 256)  # two K slices need a workspace
    x2, w2, s2 = _to_device(*_exact_case(8, 32, 512, seed=2), gpu)
    with pytest.raises(nat.FtxError) as err:
        nat.call("ftx_fp8_linear", x2.data_ptr(), w2.data_ptr(), s2.data_ptr(), y.data_ptr(), 8, 32, 512, None, 0, s)
    assert err.value.code == nat.FTX_ERR_INVALID and "workspace" in str(err.value)
    small = torch.empty(2 * 8 * 32 * 4 - 16, dtype=torch.uint8, device=gpu)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_fp8_linear", x2.data_ptr(), w2.data_ptr(), s2.data_ptr(), y.data_ptr(), 8, 32, 512,
                 small.data_ptr(), small.numel(), s)
    hip.set_fp8_linear_config(0, 0)
    with pytest.raises(nat.FtxError):
        hip.set_fp8_linear_config(9, 0)
    with pytest.raises(nat.FtxError):
        hip.set_fp8_linear_config(0, 100)
    with pytest.raises(TypeError):
        hip.fp8_linear(xt.float(), wt, st)


def test_fp8_decoder_on_gpu_matches_dequantized_float32(gpu, default_config):
    """A small fp8 decoder: decode steps (8 rows) run the kernel, the prompt (64 rows x 2) the bf16 GEMM."""
    from flextensor_amd import workloads as W

    shape = W.LlamaShape(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=300,
                         max_seq=64, fp8=True)
    model = W.build_llama(shape, seed=3)
    twin = W.build_llama(W.LlamaShape(**{**shape.__dict__, "fp8": False}), seed=0).float()
    mods = dict(model.named_modules())
    sd = {}
    for name, p in model.named_parameters():
        owner = name.rsplit(".", 1)[0]
        if isinstance(mods.get(owner), W.Fp8Linear):
            if name.endswith(".weight"):
                sd[name] = mods[owner].weight.float() * mods[owner].scale.float()[:, None]
        else:
            sd[name] = p.detach().float()
    twin.load_state_dict(sd, strict=False)
    model = model.to(gpu)
    prompt = W.prompt_tokens(8, 16, shape.vocab, seed=3)
    model.init_cache(8, 40, gpu)
    twin.init_cache(8, 40, torch.device("cpu"))
    with torch.no_grad():
        got = [model(prompt.to(gpu), 0).float().cpu()]
        want = [twin(prompt, 0)]
        tok = want[0].argmax(-1)
        for pos in range(16, 20):
            got.append(model(tok.to(gpu), pos).float().cpu())
            want.append(twin(tok, pos))
            tok = want[-1].argmax(-1)
    for g, w in zip(got, want):
        assert float((g - w).norm() / w.norm()) < REL_TOL


@pytest.mark.parametrize("m,n,k", [(0, 32, 64), (4, 0, 64), (4, 32, 0)])
def test_empty_shapes(gpu, default_config, m, n, k):
    """Empty batches and outputs launch nothing; an empty reduction gives zeros (0 * scale)."""
    from flextensor_amd import hip

    x = torch.zeros(m, k, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(n, k, dtype=torch.float8_e4m3fn, device=gpu)
    s = torch.ones(n, dtype=torch.bfloat16, device=gpu)
    y = hip.fp8_linear(x, w, s)
    torch.cuda.synchronize()
    assert y.shape == (m, n)
    assert bool((y == 0).all())


# ---- grouped launches (ftx_fp8_linear_group) --------------------------------------------------------


_GROUPS = [((96, 40, 1040), 2), ((8192, 1024, 1024), 8), ((640, 640), 8), ((300, 0, 17, 64), 5)]


@pytest.mark.parametrize("waves,slice_k", [(0, 0), (4, 256), (8, 768)])
@pytest.mark.parametrize("ns,m", _GROUPS)
def test_group_exact_products_bit_exact(gpu, default_config, ns, m, waves, slice_k):
    """Every matrix of a group matches the oracle bit for bit on exact-arithmetic data, for several launch
    shapes (one slice, split K), with empty matrices and row counts that are not multiples of 16."""
    from flextensor_amd import hip

    k = 1024
    hip.set_fp8_linear_config(waves, slice_k)
    cases = [_exact_case(m, n, k, seed=n + i) for i, n in enumerate(ns)]
    xt = _to_device(cases[0][0], cases[0][1], cases[0][2], gpu)[0]
    dev = [_to_device(cases[0][0], w_raw, scale, gpu)[1:] for _, w_raw, scale in cases]
    outs = hip.fp8_linear_group(xt, [d[0] for d in dev], [d[1] for d in dev])
    torch.cuda.synchronize()
    for (_, w_raw, scale), out, n in zip(cases, outs, ns):
        assert out.shape == (m, n)
        want = torch.from_numpy(ofp8.fp8_linear(cases[0][0], w_raw, scale)).to(torch.bfloat16)
        assert _same_values(out, want)


@pytest.mark.parametrize("ns", [(8192, 1024, 1024), (28672, 28672)])
def test_group_70b_projections_match_float64_oracle(gpu, default_config, ns):
    """The 70B layer's grouped q/k/v and gate/up calls at 8 rows, against the float64 oracle."""
    from flextensor_amd import hip

    m, k = 8, 8192
    cases = [_random_case(m, n, k, seed=n + i) for i, n in enumerate(ns)]
    xt = _to_device(*cases[0], gpu)[0]
    dev = [_to_device(cases[0][0], w_raw, scale, gpu)[1:] for _, w_raw, scale in cases]
    outs = hip.fp8_linear_group(xt, [d[0] for d in dev], [d[1] for d in dev])
    again = hip.fp8_linear_group(xt, [d[0] for d in dev], [d[1] for d in dev])
    singles = [hip.fp8_linear(xt, w, s) for w, s in dev]
    xs = xt.float().cpu().numpy()
    for (_, w_raw, _), (_, st), out, out2, one in zip(cases, dev, outs, again, singles):
        assert torch.equal(out, out2)  # deterministic
        want = torch.from_numpy(ofp8.fp8_linear(xs, w_raw, st.float().cpu().numpy()))
        got = out.double().cpu()
        assert float((got - want).norm() / want.norm()) < REL_TOL
        bound = ELEM_TOL * torch.maximum(want.abs(), want.pow(2).mean().sqrt())
        assert bool(((got - want).abs() <= bound).all())
        # against the single call: the same products, possibly another K split (fp32 rounding only)
        assert float((got - one.double().cpu()).norm() / want.norm()) < 1e-3


def test_group_graph_replays_match_eager(gpu, default_config):
    from flextensor_amd import hip

    cases = [_random_case(8, n, 4096, seed=n) for n in (2048, 512, 512)]
    xt = _to_device(*cases[0], gpu)[0]
    dev = [_to_device(cases[0][0], w_raw, scale, gpu)[1:] for _, w_raw, scale in cases]
    ws, ss = [d[0] for d in dev], [d[1] for d in dev]
    eager = hip.fp8_linear_group(xt, ws, ss)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        hip.fp8_linear_group(xt, ws, ss)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            outs = hip.fp8_linear_group(xt, ws, ss)
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, e) for o, e in zip(outs, eager)), f"replay {i}"
        assert all(torch.equal(o, e) for o, e in zip(hip.fp8_linear_group(xt, ws, ss), eager))


def test_group_rejects_bad_arguments(gpu, default_config):
    import ctypes

    from flextensor_amd import _native as nat
    from flextensor_amd import hip

    x, w_raw, scale = _exact_case(8, 32, 64, seed=1)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    with pytest.raises(ValueError):
        hip.fp8_linear_group(xt, [wt] * 5, [st] * 5)
    with pytest.raises(ValueError):
        hip.fp8_linear_group(xt, [wt, wt[:, :48].contiguous()], [st, st])
    b = ctypes.c_size_t(0)
    ns = (ctypes.c_int64 * 5)(32, 32, 32, 32, 32)
    for g in (0, 5):
        with pytest.raises(nat.FtxError) as err:
            nat.call("ftx_fp8_linear_group_workspace", 8, ctypes.cast(ns, ctypes.c_void_p), g, 64, ctypes.byref(b))
        assert err.value.code == nat.FTX_ERR_INVALID
    y = torch.empty(8, 32, dtype=torch.bfloat16, device=gpu)
    ptrs = [(ctypes.c_void_p * 2)(t.data_ptr(), 0) for t in (wt, st, y)]  # second matrix: null pointers
    with pytest.raises(nat.FtxError) as err:
        nat.call("ftx_fp8_linear_group", xt.data_ptr(), 2, *(ctypes.cast(a, ctypes.c_void_p) for a in ptrs),
                 ctypes.cast(ns, ctypes.c_void_p), 8, 64, None, 0, torch.cuda.current_stream().cuda_stream)
    assert err.value.code == nat.FTX_ERR_INVALID and "null" in str(err.value)


# ---- prefill: more than 64 rows, the tiled kernel ---------------------------------------------------


_PREFILL_SHAPES = [(65, 16, 16), (128, 128, 64), (200, 300, 528), (129, 17, 48), (512, 1024, 1024), (1000, 640, 256),
                   (300, 4100, 80)]


@pytest.mark.parametrize("m,n,k", _PREFILL_SHAPES)
def test_prefill_exact_products_bit_exact(gpu, default_config, m, n, k):
    """Tile edges in every dimension (rows, channels, K not a multiple of the 64-wide step) stay exact."""
    from flextensor_amd import hip

    x, w_raw, scale = _exact_case(m, n, k, seed=m + 3 * n + k)
    want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16)
    assert hip.fp8_linear_workspace_bytes(m, n, k) == 0  # the prefill kernel needs no workspace
    got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu))
    torch.cuda.synchronize()
    assert got.shape == (m, n)
    assert _same_values(got, want)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("m,n,k", _PREFILL_SHAPES)
def test_prefill_each_launch_shape_bit_exact(gpu, default_config, waves, m, n, k):
    """Both prefill launch shapes (4 waves / 2 LDS stages, 8 waves / 4 stages), forced, on the tile-edge cases."""
    from flextensor_amd import hip

    hip.set_fp8_linear_config(waves, 0)
    x, w_raw, scale = _exact_case(m, n, k, seed=7 * m + n + k + waves)
    want = torch.from_numpy(ofp8.fp8_linear(x, w_raw, scale)).to(torch.bfloat16)
    got = hip.fp8_linear(*_to_device(x, w_raw, scale, gpu))
    torch.cuda.synchronize()
    assert _same_values(got, want)


@pytest.mark.parametrize("m,n,k", [(512, 1024, 2048), (300, 700, 1040), (1024, 2304, 8192)])
def test_prefill_launch_shapes_agree_bitwise(gpu, default_config, m, n, k):
    """Random data: the two launch shapes accumulate every output over the same MFMA sequence."""
    from flextensor_amd import hip

    xt, wt, st = _to_device(*_random_case(m, n, k, seed=m + n), gpu)
    hip.set_fp8_linear_config(4, 0)
    y4 = hip.fp8_linear(xt, wt, st)
    hip.set_fp8_linear_config(8, 0)
    y8 = hip.fp8_linear(xt, wt, st)
    hip.set_fp8_linear_config(0, 0)
    y_auto = hip.fp8_linear(xt, wt, st)
    assert torch.equal(y4, y8)
    assert torch.equal(y4, y_auto)


@pytest.mark.parametrize("n,k", [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)])
def test_prefill_70b_shapes_match_float64_oracle(gpu, default_config, n, k):
    """512 rows (batch 8 x 64 prompt tokens) at the 70B projection shapes, against the float64 oracle."""
    from flextensor_amd import hip

    m = 512
    x, w_raw, scale = _random_case(m, n, k, seed=n + k)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    got = hip.fp8_linear(xt, wt, st)
    again = hip.fp8_linear(xt, wt, st)
    assert torch.equal(got, again)  # deterministic
    want = torch.from_numpy(ofp8.fp8_linear(xt.float().cpu().numpy(), w_raw, st.float().cpu().numpy()))
    g = got.double().cpu()
    assert float((g - want).norm() / want.norm()) < REL_TOL
    bound = ELEM_TOL * torch.maximum(want.abs(), want.pow(2).mean().sqrt())
    assert bool(((g - want).abs() <= bound).all())


def test_prefill_group_matches_single_calls(gpu, default_config):
    """A grouped prefill call (q/k/v at 512 rows) computes each matrix exactly as its single call."""
    from flextensor_amd import hip

    m, k = 512, 2048
    cases = [_random_case(m, n, k, seed=n) for n in (2048, 256, 256)]
    xt = _to_device(*cases[0], gpu)[0]
    dev = [_to_device(cases[0][0], w_raw, scale, gpu)[1:] for _, w_raw, scale in cases]
    grouped = hip.fp8_linear_group(xt, [d[0] for d in dev], [d[1] for d in dev])
    for (w, sc), y in zip(dev, grouped):
        assert torch.equal(y, hip.fp8_linear(xt, w, sc))  # same tiles, same K order


def test_prefill_weight_over_2gib_takes_the_wide_address_path(gpu, default_config):
    """A weight matrix over 2 GiB (65552 x 32768 fp8) runs the prefill kernel's 64-bit address form (the scalar-
    base form needs 31-bit offsets); sampled outputs equal exact sums of the small-integer operands."""
    from flextensor_amd import hip

    m, n, k = 80, 65552, 32768
    assert n * k >= 1 << 31
    gen = torch.Generator(device=gpu).manual_seed(9)
    mag = torch.randint(0, 3, (n, k), dtype=torch.uint8, device=gpu, generator=gen)  # |w| in {0, 1, 2}
    sign = torch.randint(0, 2, (n, k), dtype=torch.uint8, device=gpu, generator=gen)
    w_raw = torch.where(mag == 0, torch.zeros_like(mag), (0x30 + 8 * mag) | (sign << 7))  # e4m3fn 1.0 = 0x38, 2.0 = 0x40
    del sign
    x = torch.randint(-3, 4, (m, k), device=gpu, generator=gen).to(torch.bfloat16)
    scale = torch.ones(n, dtype=torch.bfloat16, device=gpu)
    y = hip.fp8_linear(x, w_raw.view(torch.float8_e4m3fn), scale)
    torch.cuda.synchronize()
    rng = np.random.default_rng(4)
    xs = x.float().cpu().numpy()
    for i, j in zip(rng.integers(0, m, 24), np.concatenate([rng.integers(0, n, 20), [0, n - 1, n - 17, 40000]])):
        wv = ofp8.decode_e4m3fn(w_raw[j].cpu().numpy())
        exact = float(np.dot(xs[i].astype(np.float64), wv))
        assert float(y[i, j].float()) == float(torch.tensor(exact).to(torch.bfloat16).float()), (i, j)
    del w_raw, mag
    torch.cuda.empty_cache()


# ---- fused epilogues: SwiGLU after gate/up, the residual add after o and down ---------------------------

_FUSED_SHAPES = [(1, 16, 16), (8, 1024, 8192), (5, 100, 48), (3, 300, 256), (17, 96, 1040), (64, 512, 256),
                 (8, 8192, 28672)]


def _fused_call(nat, x, ws, ss, epilogue, residual=None, out=None):
    """ftx_fp8_linear_fused through the C ABI; returns the output."""
    import ctypes

    m, k = x.shape
    ns = [w.shape[0] for w in ws]
    g = len(ws)
    n_arr = (ctypes.c_int64 * g)(*ns)
    b = ctypes.c_size_t(0)
    nat.call("ftx_fp8_linear_fused_workspace", m, ctypes.cast(n_arr, ctypes.c_void_p), g, k, epilogue,
             ctypes.byref(b))
    ws_buf = torch.empty(b.value, dtype=torch.uint8, device=x.device)
    y = out if out is not None else torch.empty(m, ns[0], dtype=torch.bfloat16, device=x.device)
    arrays = [(ctypes.c_void_p * g)(*[t.data_ptr() for t in ts]) for ts in (ws, ss)]
    nat.call("ftx_fp8_linear_fused", x.data_ptr(), g, *(ctypes.cast(a, ctypes.c_void_p) for a in arrays),
             y.data_ptr(), ctypes.cast(n_arr, ctypes.c_void_p), m, k, epilogue,
             residual.data_ptr() if residual is not None else None, ws_buf.data_ptr(), b.value,
             torch.cuda.current_stream(x.device).cuda_stream)
    return y, b.value


@pytest.mark.parametrize("m,n,k", _FUSED_SHAPES)
def test_residual_epilogue_is_the_linear_then_the_bf16_add(gpu, default_config, m, n, k):
    """bf16(residual + bf16(linear)): bit for bit the separate linear and torch's bf16 add, also in place
    (the residual is the output), and equal to the oracle on exact products."""
    from flextensor_amd import _native as nat
    from flextensor_amd import hip

    print(f"residual epilogue m={m} n={n} k={k}", flush=True)
    x, w_raw, scale = _random_case(m, n, k, seed=3 * m + n + k)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    resid = torch.randn(m, n, device=gpu).to(torch.bfloat16)
    want = resid + hip.fp8_linear(xt, wt, st)
    assert torch.equal(hip.fp8_linear_residual(xt, wt, st, resid), want)
    in_place = resid.clone()
    got, ws = _fused_call(nat, xt, [wt], [st], nat.FP8_EPILOGUE_RESIDUAL, residual=in_place, out=in_place)
    torch.cuda.synchronize()
    assert ws > 0 and torch.equal(got, want)
    xe, we, se = _exact_case(m, n, k, seed=m + n)
    re = np.random.default_rng(m).integers(-8, 9, size=(m, n)).astype(np.float32)
    oracle = ofp8.fp8_linear_residual(xe, we, se, re)
    got = hip.fp8_linear_residual(*_to_device(xe, we, se, gpu), torch.from_numpy(re).to(torch.bfloat16).to(gpu))
    assert _same_values(got, torch.from_numpy(oracle).to(torch.bfloat16))


def _silu_near_a_bf16_midpoint(g: torch.Tensor) -> torch.Tensor:
    """Where silu(g), in float64, lies within 2^-10 of a bf16 ulp from a rounding midpoint: the only places
    where two float32 evaluations of silu (about 2^-14 of a bf16 ulp apart) may round to different bf16
    values. ``g`` holds the bf16 gate outputs."""
    a = (g.double() / (1.0 + torch.exp(-g.double()))).abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(a.clamp_min(1e-300))) - 7)
    return ((a / ulp) % 1.0 - 0.5).abs() < 2.0 ** -10


@pytest.mark.parametrize("m,n,k", _FUSED_SHAPES)
def test_swiglu_epilogue_matches_the_oracle_and_the_separate_operations(gpu, default_config, m, n, k):
    """bf16(bf16(silu(g)) * u) against the stepwise-rounded float64 oracle on exact products, and against
    torch's F.silu(g) * u on the grouped outputs for random weights. Every output is within one bf16 ulp,
    and any that differs has its silu(g) next to a bf16 rounding midpoint, where float32 evaluations of
    silu may round either way; everywhere else the bits are equal."""
    from flextensor_amd import hip

    print(f"swiglu epilogue m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 11 + n + k)
    for exact in (True, False):
        if exact:
            xg, wg, sg = _exact_case(m, n, k, seed=m + 2 * n + k)
            _, wu, su = _exact_case(m, n, k, seed=m + 3 * n + k)
        else:
            xg, wg, sg = _random_case(m, n, k, seed=int(rng.integers(1 << 30)))
            _, wu, su = _random_case(m, n, k, seed=int(rng.integers(1 << 30)))
        xt, wgt, sgt = _to_device(xg, wg, sg, gpu)
        _, wut, sut = _to_device(xg, wu, su, gpu)
        got = hip.fp8_linear_swiglu(xt, wgt, sgt, wut, sut).double().cpu()
        g, u = hip.fp8_linear_group(xt, [wgt, wut], [sgt, sut])
        if exact:
            xf = xt.float().cpu().numpy()
            want = torch.from_numpy(ofp8.fp8_linear_swiglu(xf, wg, sgt.float().cpu().numpy(), wu,
                                                           sut.float().cpu().numpy()))
            assert _same_values(g, torch.from_numpy(ofp8.fp8_linear(xf, wg, sgt.float().cpu().numpy())).to(
                torch.bfloat16))  # the gate itself is exact
        else:
            want = (torch.nn.functional.silu(g) * u).double().cpu()
        ulp = want.abs() * 2.0 ** -7 + 1e-30
        assert bool(((got - want).abs() <= ulp).all()), f"exact={exact}"
        differ = got != want
        near = _silu_near_a_bf16_midpoint(g.cpu())
        assert not bool((differ & ~near).any()), f"exact={exact}: {int(differ.sum())} differ, " \
                                                  f"{int((differ & ~near).sum())} away from a midpoint"


def test_fused_epilogues_with_one_k_slice_and_in_graphs(gpu, default_config):
    """A call with one K slice still goes through the partials (the reduce applies the epilogue), and a
    captured graph of fused calls replays to the eager results."""
    from flextensor_amd import hip

    x, wg, sg = _random_case(4, 64, 256, seed=1)
    _, wu, su = _random_case(4, 64, 256, seed=2)
    xt, wgt, sgt = _to_device(x, wg, sg, gpu)
    _, wut, sut = _to_device(x, wu, su, gpu)
    resid = torch.randn(4, 64, device=gpu).to(torch.bfloat16)
    assert hip.fp8_linear_fused_workspace_bytes(4, [64], 256, 2) > 0
    assert torch.equal(hip.fp8_linear_residual(xt, wgt, sgt, resid), resid + hip.fp8_linear(xt, wgt, sgt))
    eager = (hip.fp8_linear_swiglu(xt, wgt, sgt, wut, sut), hip.fp8_linear_residual(xt, wgt, sgt, resid))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        hip.fp8_linear_swiglu(xt, wgt, sgt, wut, sut)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            static = (hip.fp8_linear_swiglu(xt, wgt, sgt, wut, sut), hip.fp8_linear_residual(xt, wgt, sgt, resid))
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static[0], eager[0]) and torch.equal(static[1], eager[1])
    del graph


def test_fused_rejects_bad_arguments(gpu, default_config):
    import ctypes

    from flextensor_amd import _native as nat
    from flextensor_amd import hip

    x, w_raw, scale = _random_case(8, 64, 256, seed=4)
    xt, wt, st = _to_device(x, w_raw, scale, gpu)
    resid = torch.zeros(8, 64, dtype=torch.bfloat16, device=gpu)
    n2 = (ctypes.c_int64 * 2)(64, 64)
    b = ctypes.c_size_t(0)
    cases = {
        "SwiGLU with one matrix": (8, [64], nat.FP8_EPILOGUE_SWIGLU, nat.FTX_ERR_INVALID),
        "SwiGLU with unequal n": (8, [64, 32], nat.FP8_EPILOGUE_SWIGLU, nat.FTX_ERR_INVALID),
        "residual with two matrices": (8, [64, 64], nat.FP8_EPILOGUE_RESIDUAL, nat.FTX_ERR_INVALID),
        "unknown epilogue": (8, [64], 7, nat.FTX_ERR_INVALID),
        "prefill rows": (65, [64], nat.FP8_EPILOGUE_RESIDUAL, nat.FTX_ERR_UNSUPPORTED),
    }
    for case, (m, ns, epi, code) in cases.items():
        arr = (ctypes.c_int64 * len(ns))(*ns)
        rc = nat.lib().ftx_fp8_linear_fused_workspace(m, ctypes.cast(arr, ctypes.c_void_p), len(ns), 256, epi,
                                                      ctypes.byref(b))
        assert rc == code, case
    del n2
    with pytest.raises(nat.FtxError, match="needs a residual"):
        _fused_call(nat, xt, [wt], [st], nat.FP8_EPILOGUE_RESIDUAL, residual=None)
    with pytest.raises(nat.FtxError, match="not device memory"):
        _fused_call(nat, xt, [wt], [st], nat.FP8_EPILOGUE_RESIDUAL, residual=resid.cpu())
    with pytest.raises(ValueError, match="residual must be"):
        hip.fp8_linear_residual(xt, wt, st, resid[:, :32])
    with pytest.raises(ValueError, match="decode kernel"):
        hip.fp8_linear_residual(torch.zeros(65, 256, dtype=torch.bfloat16, device=gpu), wt, st,
                                torch.zeros(65, 64, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="differ in shape"):
        hip.fp8_linear_swiglu(xt, wt, st, wt[:32].contiguous(), st[:32].contiguous())
    torch.cuda.synchronize()


def test_decoder_layer_fused_path_against_the_separate_operations(gpu, default_config, monkeypatch):
    """A 70B-shaped fp8 decoder layer at batch 8, one decode token: with the fused SwiGLU and residual
    epilogues, and with each fold switched off. Folding only the residual adds changes no bit; folding
    SwiGLU changes at most the float32 rounding of silu, so the layer stays within 1e-2 of the separate
    operations. Hooks on a projection (as the unit checks use) make the layer call that module instead."""
    from flextensor_amd import workloads as W

    s = W.LlamaShape(**{**W.LLAMA_70B_FP8.__dict__, "n_layers": 1, "vocab": 64, "max_seq": 16})
    model = W.build_llama(s, seed=3, init_device="cuda").to(gpu)
    model.init_cache(8, 8, gpu)
    layer = model.layers[0]
    x = (torch.randn(8, 1, s.hidden, device=gpu) * 0.5).to(torch.bfloat16)

    def run():
        with torch.no_grad():
            return layer(x, 3, model.rope_cos, model.rope_sin, model.cache_k[0], model.cache_v[0])

    calls = {"swiglu": 0, "residual": 0}
    real_sw, real_res = W.fp8_swiglu, W.fp8_residual
    monkeypatch.setattr(W, "fp8_swiglu", lambda *a: calls.__setitem__("swiglu", calls["swiglu"] + 1) or real_sw(*a))
    monkeypatch.setattr(W, "fp8_residual",
                        lambda *a: calls.__setitem__("residual", calls["residual"] + 1) or real_res(*a))
    fused = run()
    assert calls == {"swiglu": 1, "residual": 2}
    monkeypatch.setattr(W, "fp8_residual", lambda *a: None)
    no_residual = run()
    monkeypatch.setattr(W, "fp8_swiglu", lambda *a: None)
    separate = run()
    monkeypatch.setattr(W, "fp8_swiglu", real_sw)
    monkeypatch.setattr(W, "fp8_residual", real_res)
    assert torch.equal(no_residual, fused)  # the residual folds change no bit
    assert float((fused.double() - separate.double()).norm() / separate.double().norm()) < 1e-2
    seen = []
    handle = layer.down.register_forward_hook(lambda mod, args, out: seen.append(out))
    hooked = run()
    handle.remove()
    assert len(seen) == 1 and torch.equal(hooked, fused)
    del model
    torch.cuda.empty_cache()
