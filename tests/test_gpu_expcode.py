"""GPU decode of exponent-coded blocks, bit for bit against the raw bytes and the oracle's decoder.

The decode kernel reads the encoded block over the link from a pinned, device-mapped arena and writes
the raw bytes; every case compares the device bytes with the raw block (and, where the block is small,
with ``oracle.expcode.decode`` of the same encoded bytes).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import expcode as oxc
from oracle import expcode_dense as oxd

pytestmark = pytest.mark.gpu


def _bf16_bytes(n: int, seed: int, std: float = 0.02) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n // 2 + 1, generator=g) * std).to(torch.bfloat16).view(torch.uint8).numpy()[:n].copy()


def _specials(n: int, seed: int) -> np.ndarray:
    """bf16 words of every class: zeros, subnormals, normals over the whole range, infinities, NaNs."""
    rng = np.random.default_rng(seed)
    words = rng.integers(0, 1 << 16, size=n // 2 + 1, dtype=np.uint32)
    pick = rng.integers(0, 6, size=words.size)
    words = np.where(pick == 0, words & 0x8000, words)                 # +-0
    words = np.where(pick == 1, words & 0x807F, words)                 # subnormals
    words = np.where(pick == 2, (words & 0x8000) | 0x7F80, words)      # +-inf
    words = np.where(pick == 3, (words & 0x807F) | 0x7F81, words)      # NaNs
    return words.astype("<u2").view(np.uint8)[:n].copy()


def _raw_tensor(data: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(data.copy()) if data.size else torch.empty(0, dtype=torch.uint8)


@pytest.fixture(params=[False, True], ids=["v1", "dense"])
def dense(request):
    """Every test runs on both formats: version 1 and the dense version 2 (its link variant)."""
    return request.param


def _fmt(dense: bool):
    return oxd if dense else oxc


def _decode(raw: np.ndarray, gpu, grid: int = 0, pad: int = 0, dense: bool = False) -> tuple[np.ndarray, object]:
    from flextensor_amd import _native as nat
    from flextensor_amd import expcode

    block = expcode.encode(_raw_tensor(raw), dense=dense)
    dst = torch.full((raw.size + 2 * pad + 16,), 0xA5, dtype=torch.uint8, device=gpu)
    policy = nat.copy_policy(0, 2**63 - 1, 1, grid) if grid else None
    expcode.decode_h2d(dst[pad:], block, policy=policy)
    torch.cuda.synchronize()
    return dst.cpu().numpy(), block


@pytest.mark.parametrize("n", [1, 2, 3, 2046, 2047, 2048, 2049, 4096 * 3 + 1, (1 << 20) + 7, 64 << 20])
def test_bf16_blocks_decode_bit_exact(gpu, n, dense):
    raw = _bf16_bytes(n, seed=n)
    out, block = _decode(raw, gpu, dense=dense)
    assert np.array_equal(out[:n], raw)
    assert np.all(out[n:] == 0xA5)  # nothing past the raw size is written
    if n <= 1 << 20:
        assert _fmt(dense).decode(block.tensor.numpy()) == raw.tobytes()
    if n >= 1 << 20:
        assert block.ratio < (0.70 if dense else 0.76)


@pytest.mark.parametrize("grid", [1, 3, 8, 16, 64])
def test_every_grid_decodes_the_same_bytes(gpu, grid, dense):
    raw = _bf16_bytes((8 << 20) + 2, seed=5)
    out, _ = _decode(raw, gpu, grid=grid, dense=dense)
    assert np.array_equal(out[: raw.size], raw)


@pytest.mark.parametrize("maker", [_specials, lambda n, s: np.random.default_rng(s).integers(0, 256, n, dtype=np.uint8)])
@pytest.mark.parametrize("n", [4097, (1 << 20) + 1])
def test_escape_heavy_blocks_decode_bit_exact(gpu, maker, n, dense):
    """Blocks where many words are escapes (all exponents in use): the escape lists are long, the
    encoded block larger than the raw one, and the decode still exact."""
    raw = maker(n, 17)
    out, block = _decode(raw, gpu, dense=dense)
    assert np.array_equal(out[:n], raw)
    assert _fmt(dense).decode(block.tensor.numpy()) == raw.tobytes()


def test_decode_into_an_offset_leaves_the_rest_untouched(gpu, dense):
    raw = _bf16_bytes(100_001, seed=9)
    out, _ = _decode(raw, gpu, pad=4096, dense=dense)
    assert np.all(out[:4096] == 0xA5)
    assert np.array_equal(out[4096: 4096 + raw.size], raw)
    assert np.all(out[4096 + raw.size:] == 0xA5)


def test_graph_replays_decode_every_time(gpu, dense):
    from flextensor_amd import expcode

    raw = _bf16_bytes((4 << 20) + 6, seed=21)
    block = expcode.encode(_raw_tensor(raw), dense=dense)
    dst = torch.zeros(raw.size, dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        expcode.decode_h2d(dst, block)
    for _ in range(3):
        dst.fill_(0x3C)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy(), raw)


def test_a_captured_decode_reads_the_block_as_reencoded(gpu, dense):
    """The decode kernel reads the block's header when it runs: a graph captured before the block was
    re-encoded in place with other contents (another table, other escapes) writes the new bytes."""
    from flextensor_amd import expcode

    n = (2 << 20) + 2
    first = _bf16_bytes(n, seed=31)
    second = _bf16_bytes(n, seed=32, std=3.0)
    second[100:300] = _specials(200, 5)
    block = expcode.encode(_raw_tensor(first), capacity=n + 65536, dense=dense)
    dst = torch.zeros(n, dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        expcode.decode_h2d(dst, block)
    graph.replay()
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), first)
    table_before = bytes(block.tensor[32:72].numpy())  # escape counts and tables, in either format
    block.reencode(_raw_tensor(second))
    assert bytes(block.tensor[32:72].numpy()) != table_before
    graph.replay()
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), second)
    with pytest.raises(ValueError):
        block.reencode(_raw_tensor(second[:-2]))  # another raw size


def test_refusals_happen_on_the_host(gpu, dense):
    from flextensor_amd import _native as nat
    from flextensor_amd import expcode
    from flextensor_amd.hip import current_stream

    raw = _bf16_bytes(4 << 20, seed=3)
    block = expcode.encode(_raw_tensor(raw), dense=dense)
    s = current_stream(gpu).handle
    dst = torch.zeros(raw.size + 64, dtype=torch.uint8, device=gpu)

    def code(*args) -> int:
        with pytest.raises(nat.FtxError) as err:
            nat.call("ftx_expcode_decode_h2d", *args)
        return err.value.code

    assert code(dst.data_ptr() + 1, block.arena.ptr, block.nbytes, None, s) == nat.FTX_ERR_INVALID  # unaligned
    small = ctypes.c_void_p()  # a 2 MiB allocation asked to hold the 4 MiB block
    nat.call("ftx_device_alloc", 2 << 20, ctypes.byref(small))
    try:
        assert code(small.value, block.arena.ptr, block.nbytes, None, s) == nat.FTX_ERR_INVALID
    finally:
        nat.call("ftx_device_free", small.value)
    with pytest.raises(ValueError):
        expcode.decode_h2d(dst[: raw.size - 2], block)
    assert code(dst.data_ptr(), block.arena.ptr, block.nbytes - 4, None, s) == nat.FTX_ERR_INVALID  # truncated
    pageable = block.tensor.clone()
    assert code(dst.data_ptr(), pageable.data_ptr(), block.nbytes, None, s) == nat.FTX_ERR_UNSUPPORTED
    bad = expcode.encode(_raw_tensor(raw), dense=dense)
    bad.tensor[0] ^= 0xFF  # magic
    assert code(dst.data_ptr(), bad.arena.ptr, bad.nbytes, None, s) == nat.FTX_ERR_INVALID
    torch.cuda.synchronize()
    assert torch.count_nonzero(dst).item() == 0  # nothing ran
