"""GPU parity of the C-ABI copy engines, scatter kernel and checksum.

Every result is compared byte for byte with the CPU oracle on the same seeded
inputs (bit-exact is the bar for byte work).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native as onat

pytestmark = pytest.mark.gpu


def _rand_bytes(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, 256, size=n, dtype=np.uint8)


def _arena_with(data: np.ndarray, pad: int = 0):
    from flextensor_amd.hip import HostArena

    arena = HostArena(max(1, data.nbytes + pad + 64))
    view = arena.tensor.numpy()
    view[pad : pad + data.nbytes] = data
    return arena


@pytest.mark.parametrize("mode", ["sdma", "kernel", "auto"])
@pytest.mark.parametrize("nbytes", [1, 15, 16, 17, 4095, 4096 + 3, (1 << 20) + 7, (64 << 20) + 5])
@pytest.mark.parametrize("offset", [0, 3, 16])
def test_copy_h2d_bit_exact(gpu, mode, nbytes, offset):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    data = _rand_bytes(nbytes, seed=nbytes + offset)
    arena = _arena_with(data, pad=offset)
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    s = current_stream(gpu)
    nat.copy_h2d(dst.data_ptr() + offset, arena.ptr + offset, nbytes, nat.COPY_MODES[mode], s.handle)
    torch.cuda.synchronize()
    out = dst.cpu().numpy()
    assert np.array_equal(out[offset : offset + nbytes], data)
    # bytes outside the copied range are untouched
    assert (out[:offset] == 0xA5).all() and (out[offset + nbytes :] == 0xA5).all()


@pytest.mark.parametrize("grid", [4, 8, 16, 17, 64])  # up to 16 workgroups reserve their CUs' LDS
@pytest.mark.parametrize("nbytes", [4095, (1 << 20) + 7, (64 << 20) + 5])
def test_kernel_copy_bit_exact_at_each_grid(gpu, grid, nbytes):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    data = _rand_bytes(nbytes, seed=grid + nbytes)
    arena = _arena_with(data, pad=3)
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    default = nat.get_copy_policy()
    policy = nat.copy_policy(0, 2**63 - 1, 1, grid)  # the grid travels with the call (ftx_copy_h2d_policy)
    nat.copy_h2d(dst.data_ptr() + 3, arena.ptr + 3, nbytes, nat.COPY_KERNEL, current_stream(gpu).handle, policy)
    torch.cuda.synchronize()
    assert nat.get_copy_policy() == default
    out = dst.cpu().numpy()
    assert np.array_equal(out[3 : 3 + nbytes], data)
    assert (out[:3] == 0xA5).all() and (out[3 + nbytes :] == 0xA5).all()


@pytest.mark.parametrize("nbytes", [4095, (1 << 20) + 7, (64 << 20) + 5])
def test_auto_copy_under_a_per_call_policy_takes_the_kernel_up_to_its_cut(gpu, nbytes):
    """``FTX_COPY_AUTO`` under a caller's policy: chunks up to its kernel cut go to the zero-copy kernel at its
    grid (a link-bound ring's policy: cut at the largest unit, 8 workgroups), larger ones to SDMA; bit-exact
    either way, and the library default is untouched."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    data = _rand_bytes(nbytes, seed=nbytes ^ 0x5A)
    arena = _arena_with(data, pad=16)
    default = nat.get_copy_policy()
    for cut in (nbytes, nbytes - 1):  # kernel, then SDMA
        dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
        policy = nat.copy_policy(cut, 2**63 - 1, 1, 8)
        nat.copy_h2d(dst.data_ptr() + 16, arena.ptr + 16, nbytes, nat.COPY_AUTO, current_stream(gpu).handle, policy)
        torch.cuda.synchronize()
        out = dst.cpu().numpy()
        assert np.array_equal(out[16: 16 + nbytes], data), cut
        assert (out[:16] == 0xA5).all() and (out[16 + nbytes:] == 0xA5).all()
    assert nat.get_copy_policy() == default


def test_kernel_copy_rejects_non_congruent_alignment(gpu):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    data = _rand_bytes(4096, seed=7)
    arena = _arena_with(data)
    dst = torch.zeros(8192, dtype=torch.uint8, device=gpu)
    s = current_stream(gpu)
    with pytest.raises(nat.FtxError) as err:
        nat.copy_h2d(dst.data_ptr() + 1, arena.ptr, 4096, nat.COPY_KERNEL, s.handle)
    assert err.value.code == nat.FTX_ERR_UNSUPPORTED
    # AUTO falls back to SDMA for the same request and stays bit-exact
    nat.copy_h2d(dst.data_ptr() + 1, arena.ptr, 4096, nat.COPY_AUTO, s.handle)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy()[1:4097], data)


@pytest.mark.parametrize("per_call", [True, False])
def test_split_sdma_over_copy_streams(gpu, per_call):
    """SDMA split over four copy streams, under a per-call policy and under the library default."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    old = nat.get_copy_policy()
    policy = nat.copy_policy(1 << 20, 1 << 20, 4, 0)
    try:
        if not per_call:
            nat.set_copy_policy(*policy.astuple())
        n = (48 << 20) + 333
        data = _rand_bytes(n, seed=11)
        arena = _arena_with(data)
        for mode in (nat.COPY_SDMA, nat.COPY_AUTO):
            dst = torch.zeros(n, dtype=torch.uint8, device=gpu)
            nat.copy_h2d(dst.data_ptr(), arena.ptr, n, mode, current_stream(gpu).handle,
                         policy if per_call else None)
            torch.cuda.synchronize()
            assert np.array_equal(dst.cpu().numpy(), data)
    finally:
        nat.set_copy_policy(*old)


def test_split_sdma_from_two_host_threads(gpu):
    """Split copies made from two host threads at once, each on its own stream right after a fill of its
    destination. The split copies of a device share their fork and join events, so each copy's pieces must
    still start after its own stream's fill: every destination ends up holding its own source bytes."""
    import threading

    from flextensor_amd import _native as nat
    from flextensor_amd.hip import new_stream

    policy = nat.copy_policy(0, 1 << 20, 4, 0)
    n = (24 << 20) + 77
    datas = [_rand_bytes(n, seed=40 + i) for i in range(2)]
    arenas = [_arena_with(d) for d in datas]
    dsts = [torch.empty(n, dtype=torch.uint8, device=gpu) for _ in range(2)]
    streams = [new_stream(gpu) for _ in range(2)]
    torch.cuda.synchronize()
    start = threading.Barrier(2)
    errors: list[BaseException] = []

    def worker(i: int) -> None:
        try:
            start.wait()
            for _ in range(20):
                nat.call("ftx_memset_async", dsts[i].data_ptr(), 0x5A, n, streams[i].handle)
                nat.copy_h2d(dsts[i].data_ptr(), arenas[i].ptr, n, nat.COPY_SDMA, streams[i].handle, policy)
        except BaseException as exc:  # reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for dst, data in zip(dsts, datas):
        assert np.array_equal(dst.cpu().numpy(), data)


def _scatter_case(seed: int, n_desc: int, max_bytes: int, align_dst: bool):
    rng = np.random.default_rng(seed)
    sizes = np.exp(rng.uniform(np.log(1), np.log(max_bytes), size=n_desc)).astype(np.int64)
    sizes[rng.integers(0, n_desc, size=max(1, n_desc // 10))] = 0  # empty descriptors
    offsets, total = onat.packed_layout(sizes.tolist(), 128)
    chunk = _rand_bytes(max(total, 1), seed=seed + 1)
    return sizes, offsets, chunk


@pytest.mark.parametrize("seed,n_desc,max_bytes", [(1, 1, 4096), (2, 37, 70000), (3, 500, 1 << 20), (4, 2000, 200000)])
@pytest.mark.parametrize("tile", [None, 0, 1040, 4096, 65536])  # None: one-shot ftx_scatter; 0: default tile
def test_scatter_matches_oracle(gpu, seed, n_desc, max_bytes, tile):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    sizes, offsets, chunk = _scatter_case(seed, n_desc, max_bytes, True)
    chunk_dev = torch.from_numpy(chunk).to(gpu)
    rng = np.random.default_rng(seed + 2)
    # destinations: separate device tensors, some at odd byte offsets
    shifts = rng.integers(0, 4, size=n_desc) * np.array([0, 1, 4, 16])[rng.integers(0, 4, size=n_desc)] % 64
    dsts = [torch.full((int(n) + 80,), 0x5A, dtype=torch.uint8, device=gpu) for n in sizes]
    descs = [(off, d.data_ptr() + int(sh), int(n)) for off, d, sh, n in zip(offsets, dsts, shifts, sizes)]
    arr = nat.make_desc_array(descs)
    s = current_stream(gpu)
    if tile is not None:
        import ctypes

        plan = ctypes.c_void_p()
        nat.call("ftx_scatter_plan_create", arr, len(descs), tile, ctypes.byref(plan))
        try:
            nat.call("ftx_scatter_run", plan, chunk_dev.data_ptr(), s.handle)
            torch.cuda.synchronize()
        finally:
            nat.call("ftx_scatter_plan_destroy", plan)
    else:
        nat.call("ftx_scatter", chunk_dev.data_ptr(), arr, len(descs), s.handle)
        torch.cuda.synchronize()
    # oracle on host buffers with the same layout
    expect = [np.full(int(n) + 80, 0x5A, dtype=np.uint8) for n in sizes]
    onat.scatter(chunk, [(off, int(n)) for off, n in zip(offsets, sizes)],
                 [e[int(sh):] for e, sh in zip(expect, shifts)])
    for d, e in zip(dsts, expect):
        assert np.array_equal(d.cpu().numpy(), e)


@pytest.mark.parametrize("nbytes", [0, 1, 7, 8, 9, 4095, 4096, 4097, 123457, (3 << 20) + 5])
def test_checksum_matches_oracle(gpu, nbytes):
    from flextensor_amd.hip import checksum

    data = _rand_bytes(nbytes, seed=nbytes)
    t = torch.from_numpy(data.copy()).to(gpu) if nbytes else torch.empty(0, dtype=torch.uint8, device=gpu)
    assert checksum(t) == onat.checksum64(data)


def test_device_info(gpu):
    from flextensor_amd import _native as nat

    cu, xcd, mem = nat.device_info()
    print(f"device: {cu} CUs, {xcd} XCDs, {mem / 2**30:.1f} GiB")
    assert cu > 0 and xcd >= 1 and mem > 0


@pytest.mark.parametrize("mode", ["sdma", "kernel"])
def test_copy_rejects_host_destination(gpu, mode):
    """A CPU tensor as destination is rejected on the host, before any launch."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    data = _rand_bytes(1 << 16, seed=3)
    arena = _arena_with(data)
    host_dst = torch.zeros(1 << 16, dtype=torch.uint8)
    with pytest.raises(nat.FtxError) as err:
        nat.copy_h2d(host_dst.data_ptr(), arena.ptr, 1 << 16, nat.COPY_MODES[mode], current_stream(gpu).handle)
    assert err.value.code == nat.FTX_ERR_INVALID
    assert "device memory" in str(err.value)


def test_kernel_copy_rejects_source_past_arena(gpu):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HostArena, current_stream

    arena = HostArena(4096)
    dst = torch.zeros(8192, dtype=torch.uint8, device=gpu)
    with pytest.raises(nat.FtxError) as err:
        nat.copy_h2d(dst.data_ptr(), arena.ptr, 8192, nat.COPY_KERNEL, current_stream(gpu).handle)
    assert err.value.code == nat.FTX_ERR_INVALID


def test_transfer_stream_runs_beside_compute(gpu):
    """The transfer stream does not share a hardware queue with torch's compute stream."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HipEvent, HostArena, current_stream, transfer_stream

    s = transfer_stream(gpu)
    comp = current_stream(gpu)
    a = torch.randn(8192, 8192, device=gpu, dtype=torch.bfloat16)
    arena = HostArena(64 << 20)
    dst = torch.empty(64 << 20, dtype=torch.uint8, device=gpu)
    torch.matmul(a, a)  # first call at this shape selects the GEMM kernel on the host; keep that out of the window
    nat.copy_h2d(dst.data_ptr(), arena.ptr, 64 << 20, nat.COPY_SDMA, s.handle)
    torch.cuda.synchronize()
    start, gemm_end, copy_end = HipEvent(True), HipEvent(True), HipEvent(True)
    comp.record_event(start)
    for _ in range(20):
        torch.matmul(a, a)
    comp.record_event(gemm_end)
    nat.copy_h2d(dst.data_ptr(), arena.ptr, 64 << 20, nat.COPY_SDMA, s.handle)
    s.record_event(copy_end)
    torch.cuda.synchronize()
    assert start.elapsed_time(copy_end) < 0.5 * start.elapsed_time(gemm_end)
    assert transfer_stream(gpu) is s  # one per device
    from flextensor_amd.hip import transfer_stream_probe

    probe = transfer_stream_probe(gpu)
    print(f"transfer stream probe: {probe}", flush=True)
    assert probe["chosen_candidate"] == probe["rejected"] < probe["attempts"]
    assert probe["transfer_fill_done_ms"] < 0.8 * probe["compute_busy_ms"]


def test_arena_freed_by_refcount_when_last_view_dies(gpu):
    """Pinned memory is returned as soon as the last view goes (no garbage-collector cycle)."""
    import gc

    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HostArena

    gc.disable()
    try:
        a = HostArena(1 << 20)
        ptr = a.ptr
        view = a.tensor[100:200]
        view.fill_(7)
        del a
        assert nat.host_device_ptr(ptr)  # still registered: the view keeps it alive
        assert int(view.sum()) == 700
        del view
        with pytest.raises(nat.FtxError):
            nat.host_device_ptr(ptr)
    finally:
        gc.enable()


def test_device_clock_agrees_with_hip_events(gpu):
    """ftx_timestamp: kernel-written wall-clock stamps time the same span as hipEvents."""
    from flextensor_amd.hip import DeviceClock, HipEvent, current_stream

    clock = DeviceClock(2, gpu)
    a, b = clock.event(), clock.event()
    e0, e1 = HipEvent(True), HipEvent(True)
    s = current_stream(gpu)
    x = torch.randn(4096, 4096, device=gpu, dtype=torch.bfloat16)
    torch.matmul(x, x)
    torch.cuda.synchronize()
    a.record(s)
    e0.record(s)
    for _ in range(20):
        torch.matmul(x, x)
    e1.record(s)
    b.record(s)
    torch.cuda.synchronize()
    clock.refresh()
    ms_clock, ms_event = a.elapsed_time(b), e0.elapsed_time(e1)
    assert ms_event > 0.5
    assert abs(ms_clock - ms_event) <= 0.05 * ms_event + 0.05


def test_timestamp_rejects_host_slot(gpu):
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    host = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_timestamp", host.data_ptr(), current_stream(gpu).handle)


def test_probes_write_nothing_and_check_arguments(gpu):
    """The HBM read probe and the MFMA probe leave their sink alone and refuse bad arguments."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import current_stream

    s = current_stream(gpu).handle
    sink = torch.full((1,), -7, dtype=torch.int32, device=gpu)
    buf = torch.randint(0, 256, (1 << 20,), dtype=torch.uint8, device=gpu)
    nat.call("ftx_hbm_read_probe", buf.data_ptr(), buf.numel(), sink.data_ptr(), 64, s)
    nat.call("ftx_mfma_probe", 8, 16, sink.data_ptr(), s)
    nat.call("ftx_mfma_probe_shape", 1, 8, 16, sink.data_ptr(), s)
    torch.cuda.synchronize()
    assert int(sink.item()) == -7
    with pytest.raises(nat.FtxError, match="shape"):
        nat.call("ftx_mfma_probe_shape", 2, 8, 16, sink.data_ptr(), s)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_hbm_read_probe", buf.data_ptr() + 1, 64, sink.data_ptr(), 64, s)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_mfma_probe", 0, 16, sink.data_ptr(), s)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_mfma_probe", 8, 0, sink.data_ptr(), s)
    host = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(nat.FtxError):
        nat.call("ftx_mfma_probe", 8, 16, host.data_ptr(), s)


@pytest.mark.parametrize("mode", ["sdma", "kernel"])
def test_device_only_event_orders_a_copy_before_its_consumer(gpu, mode):
    """An ``FTX_EVENT_DEVICE_ONLY`` event recorded after a copy on one stream orders a kernel on another
    stream after the copy: the consumer reads every copied byte."""
    from flextensor_amd import _native as nat
    from flextensor_amd.hip import HipEvent, current_stream, new_stream

    n = (32 << 20) + 48
    data = _rand_bytes(n, seed=23)
    arena = _arena_with(data)
    dst = torch.zeros(n, dtype=torch.uint8, device=gpu)
    comp, xs = current_stream(gpu), new_stream(gpu, name="device-only-event-test")
    torch.cuda.synchronize()
    for _ in range(3):
        dst.zero_()
        xs.wait_stream(comp)
        nat.copy_h2d(dst.data_ptr(), arena.ptr, n, nat.COPY_MODES[mode], xs.handle)
        comp.wait_event(xs.record_event(HipEvent(device_only=True)))
        got = dst.clone()  # on the compute stream, after the wait
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), data)


def test_shutdown_drains_queued_copies_and_refuses_more_work(gpu):
    """``ftx_shutdown`` on a GPU, in a child process (a shut-down library stays refused for the rest of its
    process): copies queued on every engine (SDMA, SDMA split over copy streams, the zero-copy kernel, the
    staged engine with its host threads and staging buffers) have all landed when it returns, later work
    is refused with FTX_ERR_UNSUPPORTED, torch keeps working, and the process exits cleanly."""
    import subprocess
    import sys
    from pathlib import Path

    code = (
        "import torch\n"
        "import flextensor_amd._native as nat\n"
        "from flextensor_amd.hip import HostArena, current_stream\n"
        "torch.cuda.set_device(0)\n"
        "nat.load()\n"
        "dev = torch.device('cuda', 0)\n"
        "s = current_stream(dev)\n"
        "n = 96 << 20\n"
        "arena = HostArena(n)\n"
        "arena.tensor.random_(0, 256)\n"
        "pageable = torch.randint(0, 256, (n,), dtype=torch.uint8)\n"
        "split = nat.copy_policy(1 << 20, 1 << 20, 4, 0)\n"
        "outs = [torch.zeros(n, dtype=torch.uint8, device=dev) for _ in range(4)]\n"
        "torch.cuda.synchronize()\n"
        "nat.copy_h2d(outs[0].data_ptr(), arena.ptr, n, nat.COPY_SDMA, s.handle)\n"
        "nat.copy_h2d(outs[1].data_ptr(), arena.ptr, n, nat.COPY_SDMA, s.handle, split)\n"
        "nat.copy_h2d(outs[2].data_ptr(), arena.ptr, n, nat.COPY_KERNEL, s.handle)\n"
        "nat.copy_h2d(outs[3].data_ptr(), pageable.data_ptr(), n, nat.COPY_STAGED, s.handle)\n"
        "nat.shutdown()\n"
        "assert s.query(), 'work still queued after ftx_shutdown'\n"
        "host = arena.tensor.clone()\n"
        "assert all(torch.equal(o.cpu(), host) for o in outs[:3]) and torch.equal(outs[3].cpu(), pageable)\n"
        "try:\n"
        "    nat.copy_h2d(outs[0].data_ptr(), arena.ptr, n, nat.COPY_SDMA, s.handle)\n"
        "except nat.FtxError as e:\n"
        "    assert e.code == nat.FTX_ERR_UNSUPPORTED and 'shut down' in str(e)\n"
        "else:\n"
        "    raise SystemExit('a copy ran after ftx_shutdown')\n"
        "nat.shutdown()\n"
        "assert float(torch.ones(4, device=dev).sum()) == 4.0\n"
        "print('drained', flush=True)\n"
    )
    print("shutdown on the GPU: child process", flush=True)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240,
                         cwd=str(Path(__file__).resolve().parents[1]))
    assert out.returncode == 0 and out.stdout.strip().endswith("drained"), out.stdout + out.stderr
    assert "ftx_shutdown at exit returned" not in out.stderr
