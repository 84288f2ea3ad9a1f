"""The allocation-free fp8 linear entry point against the allocating one, through the C ABI, on the GPU.

``ftx_fp8_linear_static`` keeps its split-K partial sums in the library's
static per-GPU scratch array instead of a caller workspace. Its results must
be bit-identical to ``ftx_fp8_linear`` (same launch shape, same summation
order) on consecutive calls, the second smaller than the first, so stale
partials of a larger call cannot leak into a smaller one. A call whose
partials exceed the array is refused before any operand is touched.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(gen: torch.Generator, m: int, n: int, k: int, dev: torch.device):
    x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
    w = (torch.randn(n, k, device=dev, generator=gen) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
    sc = (torch.rand(n, device=dev, generator=gen) / 448 + 1e-4).to(torch.bfloat16)
    return x, w, sc


def _with_workspace(nat, x, w, sc, stream: int) -> torch.Tensor:
    m, k = x.shape
    n = w.shape[0]
    b = ctypes.c_size_t(0)
    nat.call("ftx_fp8_linear_workspace", m, n, k, ctypes.byref(b))
    ws = torch.empty(max(1, b.value), dtype=torch.uint8, device=x.device)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    nat.call("ftx_fp8_linear", x.data_ptr(), w.data_ptr(), sc.data_ptr(), y.data_ptr(), m, n, k, ws.data_ptr(),
             b.value, stream)
    return y, b.value


def test_static_scratch_entry_point_matches_the_workspace_one(gpu):
    from flextensor_amd import _native as nat

    stream = torch.cuda.current_stream(gpu).cuda_stream
    gen = torch.Generator(device=gpu).manual_seed(11)
    # a 70B down projection at batch 8 (16 K slices), then a smaller call that uses less of the scratch
    for m, n, k in ((8, 8192, 28672), (3, 1024, 4096), (8, 8192, 28672)):
        print(f"fp8 linear static: m={m} n={n} k={k}", flush=True)
        x, w, sc = _operands(gen, m, n, k, gpu)
        want, ws_bytes = _with_workspace(nat, x, w, sc, stream)
        assert ws_bytes > 0  # the call does use split-K partials
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        nat.call("ftx_fp8_linear_static", x.data_ptr(), w.data_ptr(), sc.data_ptr(), got.data_ptr(), m, n, k, stream)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_static_scratch_refuses_calls_beyond_its_size(gpu):
    from flextensor_amd import _native as nat

    b = ctypes.c_size_t(0)
    m, n, k = 64, 1 << 24, 1 << 16  # partial sums far beyond the array; no operand is read
    nat.call("ftx_fp8_linear_workspace", m, n, k, ctypes.byref(b))
    assert b.value > 64 << 20
    with pytest.raises(nat.FtxError, match="static scratch") as info:
        nat.call("ftx_fp8_linear_static", None, None, None, None, m, n, k, torch.cuda.current_stream(gpu).cuda_stream)
    assert info.value.code == nat.FTX_ERR_UNSUPPORTED


def test_python_wrapper_refuses_bad_operands_and_matches_the_entry_point(gpu):
    """``hip.fp8_linear_static`` checks its operands as ``fp8_linear`` does (dtypes, shapes, one device,
    contiguity) before the call, and otherwise returns what ``fp8_linear`` computes, bit for bit."""
    from flextensor_amd import hip

    gen = torch.Generator(device=gpu).manual_seed(5)
    m, n, k = 8, 1024, 4096
    x, w, sc = _operands(gen, m, n, k, gpu)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    assert torch.equal(hip.fp8_linear_static(x, w, sc, out), hip.fp8_linear(x, w, sc))
    bad = {
        "float32 scale": (x, w, sc.float(), out),
        "bf16 weight": (x, w.to(torch.bfloat16), sc, out),
        "weight K mismatch": (x, w[:, : k // 2].contiguous(), sc, out),
        "scale length": (x, w, sc[: n // 2], out),
        "scale on the host": (x, w, sc.cpu(), out),
        "strided scale": (x, w, torch.stack([sc, sc], 1)[:, 0], out),
        "wrong out shape": (x, w, sc, out[:, : n // 2]),
        "float32 out": (x, w, sc, out.float()),
    }
    for case, args in bad.items():
        with pytest.raises((ValueError, TypeError)):
            hip.fp8_linear_static(*args)
        print(f"fp8_linear_static refused: {case}", flush=True)
    torch.cuda.synchronize()
