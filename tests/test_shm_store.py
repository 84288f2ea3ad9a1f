"""Shared resident-tensor store: byte format, validation, materialization (CPU).

Models and corruption cases follow the reference's own store tests
(tests/unit/shm/test_shared_tensor_store.py:153-190, 206-668); the layout of
the mixed model's store is written out by hand below from the format rules,
so the offsets and the manifest are pinned byte for byte.
"""

from __future__ import annotations

import json
import multiprocessing as mp
import os
import struct

import pytest
import torch
from torch import nn

from flextensor_amd.shm import HEADER, SharedSegment, SharedTensorStore, store_segment_name


class _Mixed(nn.Module):
    """Same tensors as the reference's mixed model (test_shared_tensor_store.py:153-172)."""

    def __init__(self, device: str = "cpu", values: bool = True) -> None:
        super().__init__()
        w = torch.arange(6, dtype=torch.float32, device=device).reshape(2, 3)
        sc = torch.tensor(7.5, dtype=torch.float64, device=device)
        cnt = torch.tensor([3, 5], dtype=torch.int64, device=device)
        scr = torch.tensor([1.25, 2.5], dtype=torch.float16, device=device)
        if not values and device != "meta":
            for t in (w, sc, cnt, scr):
                t.zero_()
        self.weight = nn.Parameter(w)
        self.scalar = nn.Parameter(sc)
        self.empty = nn.Parameter(torch.empty((0, 2), dtype=torch.float32, device=device))
        self.offloaded = nn.Parameter(torch.ones(2, dtype=torch.float32, device=device))
        self.register_buffer("counter", cnt)
        self.register_buffer("scratch", scr, persistent=False)
        self.register_buffer("optional", None)
        self.unregistered = torch.tensor([99], device=device)


class _Alias(nn.Module):
    def __init__(self, tied: bool = True, device: str = "cpu") -> None:
        super().__init__()
        left = nn.Parameter(torch.arange(4, dtype=torch.float32, device=device).reshape(2, 2))
        self.left = left
        self.right = left if tied else nn.Parameter(torch.zeros((2, 2), dtype=torch.float32, device=device))
        first = torch.tensor([4, 8], dtype=torch.int32, device=device)
        self.register_buffer("first", first)
        self.register_buffer("second", first if tied else torch.zeros(2, dtype=torch.int32, device=device))


@pytest.fixture
def ns(request):
    name = f"ftx_{os.getpid()}_{request.node.name}".replace("[", "_").replace("]", "").replace("-", "_")[:200]
    yield name
    try:
        os.unlink(os.path.join("/dev/shm", store_segment_name(name)))
    except FileNotFoundError:
        pass


def _raw(ns: str) -> SharedSegment:
    return SharedSegment(store_segment_name(ns))


def _rewrite_manifest(ns: str, edit) -> None:
    seg = _raw(ns)
    buf = seg.buf
    magic, version, mlen, data_offset, data_size = HEADER.unpack_from(buf, 0)
    manifest = json.loads(bytes(buf[HEADER.size:HEADER.size + mlen]))
    edit(manifest)
    enc = json.dumps(manifest, sort_keys=True, separators=(",", ":")).encode()
    assert len(enc) <= data_offset - HEADER.size
    buf[HEADER.size:HEADER.size + len(enc)] = enc
    HEADER.pack_into(buf, 0, magic, version, len(enc), data_offset, data_size)
    seg.close()


# ---- byte layout pinned by hand ------------------------------------------------------


def test_mixed_store_bytes_match_the_format_rules(ns):
    src = _Mixed()
    store = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight", "scalar", "empty"])
    try:
        seg = _raw(ns)
        buf = bytes(seg.buf)
        seg.close()
        magic, version, mlen, data_offset, data_size = struct.unpack_from("<4sIQQQ", buf, 0)
        assert (magic, version) == (b"FTTS", 1) and HEADER.size == 32
        # parameters in request order, then buffers; offsets aligned to max(8, itemsize)
        # weight f32[2,3] 24 B @0; scalar f64 8 B @24; empty 0 B @32; counter i64[2] 16 B @32; scratch f16[2] 4 B @48
        want = {"tensors": [
            {"aliases": ["weight"], "dtype": "float32", "kind": "parameter", "payload_offset": 0, "persistent": None,
             "requires_grad": True, "shape": [2, 3], "stride": [3, 1]},
            {"aliases": ["scalar"], "dtype": "float64", "kind": "parameter", "payload_offset": 24, "persistent": None,
             "requires_grad": True, "shape": [], "stride": []},
            {"aliases": ["empty"], "dtype": "float32", "kind": "parameter", "payload_offset": 32, "persistent": None,
             "requires_grad": True, "shape": [0, 2], "stride": [2, 1]},
            {"aliases": ["counter"], "dtype": "int64", "kind": "buffer", "payload_offset": 32, "persistent": [True],
             "requires_grad": False, "shape": [2], "stride": [1]},
            {"aliases": ["scratch"], "dtype": "float16", "kind": "buffer", "payload_offset": 48, "persistent": [False],
             "requires_grad": False, "shape": [2], "stride": [1]},
        ]}
        enc = json.dumps(want, sort_keys=True, separators=(",", ":")).encode()
        assert buf[32:32 + mlen] == enc and mlen == len(enc)
        assert data_offset == -(-(32 + mlen) // 64) * 64 and data_size == 52
        d = buf[data_offset:data_offset + data_size]
        assert d[0:24] == src.weight.detach().numpy().tobytes()
        assert d[24:32] == struct.pack("<d", 7.5)
        assert d[32:48] == struct.pack("<qq", 3, 5)
        assert d[48:52] == src.scratch.numpy().tobytes()
        assert len(buf) == data_offset + data_size
    finally:
        store.close()


# ---- the reference's cases ----------------------------------------------------------


def test_mixed_roundtrip_and_copy_out(ns):
    # test_shared_tensor_store.py:206-228
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight", "scalar", "empty"])
    follower = SharedTensorStore.attach(ns)
    target = _Mixed(device="meta")
    follower.materialize_into(target, device="cpu")
    follower.close()
    creator.close()
    torch.testing.assert_close(target.weight, src.weight)
    torch.testing.assert_close(target.scalar, src.scalar)
    assert target.empty.shape == (0, 2)
    torch.testing.assert_close(target.counter, src.counter)
    torch.testing.assert_close(target.scratch, src.scratch)
    assert "scratch" in target._non_persistent_buffers_set
    assert target.offloaded.device.type == "meta" and target.unregistered.device.type == "meta"
    assert not os.path.exists(os.path.join("/dev/shm", store_segment_name(ns)))


def test_page_rounded_trailing_bytes_accepted(ns):
    # test_shared_tensor_store.py:231-245
    from flextensor_amd.shm import read_manifest

    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    try:
        seg = _raw(ns)
        logical = bytes(seg.buf)
        seg.close()
        padded = memoryview(logical + bytes(4096))
        descs, data_offset = read_manifest(padded)
        padded.release()
        assert data_offset < len(logical)
        assert {d.aliases[0] for d in descs} == {"weight", "counter", "scratch"}
    finally:
        creator.close()


def test_meta_placeholder_takes_stored_dtype(ns):
    # test_shared_tensor_store.py:248-262
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    follower = SharedTensorStore.attach(ns)
    target = _Mixed(device="meta")
    target.weight = nn.Parameter(torch.empty(src.weight.shape, dtype=torch.bfloat16, device="meta"))
    follower.materialize_into(target, device="cpu")
    follower.close()
    creator.close()
    assert target.weight.dtype == torch.float32
    torch.testing.assert_close(target.weight, src.weight)


@pytest.mark.parametrize("dtype_name", ["float32", "float", "", "bogus", "Tensor", None, False, 42])
def test_manifest_dtype_validation(ns, dtype_name):
    # test_shared_tensor_store.py:265-291
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    try:
        _rewrite_manifest(ns, lambda m: m["tensors"][0].__setitem__("dtype", dtype_name))
        if dtype_name in {"float32", "float"}:
            follower = SharedTensorStore.attach(ns)
            target = _Mixed(device="meta")
            follower.materialize_into(target, device="cpu")
            follower.close()
            torch.testing.assert_close(target.weight, src.weight)
        else:
            with pytest.raises(RuntimeError, match=r"manifest.*dtype"):
                SharedTensorStore.attach(ns)
    finally:
        creator.close()


def test_dense_transpose_keeps_layout(ns):
    # test_shared_tensor_store.py:356-372
    src = nn.Module()
    src.weight = nn.Parameter(torch.arange(12, dtype=torch.float32).reshape(3, 4).t())
    target = nn.Module()
    target.weight = nn.Parameter(torch.empty_strided(src.weight.shape, src.weight.stride(), device="meta"))
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    follower = SharedTensorStore.attach(ns)
    follower.materialize_into(target, device="cpu")
    torch.testing.assert_close(target.weight, src.weight)
    assert target.weight.stride() == src.weight.stride()
    follower.close()
    creator.close()


@pytest.mark.parametrize("make", [lambda: torch.arange(8, dtype=torch.float32).as_strided((2, 3), (4, 1)),
                                  lambda: torch.arange(9, dtype=torch.float32).as_strided((3, 3), (2, 2))],
                         ids=["gapped", "overlapping"])
def test_non_dense_layout_stored_contiguous(ns, make):
    # test_shared_tensor_store.py:375-406
    src = nn.Module()
    src.weight = nn.Parameter(make())
    target = nn.Module()
    target.weight = nn.Parameter(torch.empty(tuple(src.weight.shape), dtype=torch.float32, device="meta"))
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    follower = SharedTensorStore.attach(ns)
    follower.materialize_into(target, device="cpu")
    torch.testing.assert_close(target.weight, src.weight)
    assert target.weight.is_contiguous()
    follower.close()
    creator.close()


def test_aliases_share_one_payload(ns):
    # test_shared_tensor_store.py:409-425
    src = _Alias()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["left"])
    seg = _raw(ns)
    _, _, mlen, _, _ = HEADER.unpack_from(seg.buf, 0)
    manifest = json.loads(bytes(seg.buf[HEADER.size:HEADER.size + mlen]))
    seg.close()
    follower = SharedTensorStore.attach(ns)
    target = _Alias(tied=False, device="meta")
    follower.materialize_into(target, device="cpu")
    assert len(manifest["tensors"]) == 2
    assert manifest["tensors"][0]["aliases"] == ["left", "right"]
    assert target.left is target.right and target.first is target.second
    torch.testing.assert_close(target.left, src.left)
    torch.testing.assert_close(target.first, src.first)
    follower.close()
    creator.close()


def test_buffer_persistence_from_manifest(ns):
    # test_shared_tensor_store.py:428-442
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=[])
    follower = SharedTensorStore.attach(ns)
    target = _Mixed(values=False)
    target._non_persistent_buffers_set.discard("scratch")
    follower.materialize_into(target, device="cpu")
    assert "scratch" in target._non_persistent_buffers_set
    torch.testing.assert_close(target.scratch, src.scratch)
    follower.close()
    creator.close()


@pytest.mark.parametrize("requested", [["missing"], ["counter"]])
def test_creator_rejects_missing_or_buffer_names(ns, requested):
    # test_shared_tensor_store.py:445-450
    with pytest.raises(ValueError, match=requested[0]):
        SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=requested)
    assert not os.path.exists(os.path.join("/dev/shm", store_segment_name(ns)))


def test_creator_rejects_sparse(ns):
    # test_shared_tensor_store.py:453-460
    m = nn.Module()
    m.weight = nn.Parameter(torch.sparse_coo_tensor(torch.tensor([[0]]), torch.tensor([1.0]), (2,)))
    with pytest.raises(ValueError, match="strided"):
        SharedTensorStore.create_from_model(ns, m, parameter_names=["weight"])


def test_validation_before_any_mutation(ns):
    # test_shared_tensor_store.py:463-486
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight", "scalar"])
    follower = SharedTensorStore.attach(ns)
    target = _Mixed(values=False)
    w0, c0 = target.weight, target.counter
    target.scalar = nn.Parameter(torch.zeros((), dtype=torch.float32))
    with pytest.raises(ValueError, match=r"scalar.*dtype"):
        follower.materialize_into(target, device="cpu")
    assert target.weight is w0 and target.counter is c0
    assert torch.count_nonzero(target.weight) == 0 and torch.count_nonzero(target.counter) == 0
    follower.close()
    creator.close()


@pytest.mark.parametrize("offset,replacement,message", [(0, b"NOPE", "magic"), (4, struct.pack("<I", 99), "version")])
def test_attach_rejects_bad_magic_or_version(ns, offset, replacement, message):
    # test_shared_tensor_store.py:489-505
    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    seg = _raw(ns)
    seg.buf[offset:offset + len(replacement)] = replacement
    seg.close()
    with pytest.raises(RuntimeError, match=message):
        SharedTensorStore.attach(ns)
    creator.close()


def test_attach_rejects_invalid_json(ns):
    # test_shared_tensor_store.py:508-518
    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    seg = _raw(ns)
    seg.buf[HEADER.size] = ord("!")
    seg.close()
    with pytest.raises(RuntimeError, match="manifest"):
        SharedTensorStore.attach(ns)
    creator.close()


@pytest.mark.parametrize("field", ["manifest_length", "data_offset", "data_size"])
def test_attach_rejects_header_bounds(ns, field):
    # test_shared_tensor_store.py:544-561
    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    seg = _raw(ns)
    magic, version, mlen, data_offset, data_size = HEADER.unpack_from(seg.buf, 0)
    n = seg.size
    if field == "manifest_length":
        mlen = n
    elif field == "data_offset":
        data_offset = HEADER.size
    else:
        data_size = n
    HEADER.pack_into(seg.buf, 0, magic, version, mlen, data_offset, data_size)
    seg.close()
    with pytest.raises(RuntimeError, match="bounds"):
        SharedTensorStore.attach(ns)
    creator.close()


def test_attach_rejects_payload_outside_data(ns):
    # test_shared_tensor_store.py:564-581
    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    seg = _raw(ns)
    data_size = HEADER.unpack_from(seg.buf, 0)[4]
    seg.close()
    _rewrite_manifest(ns, lambda m: m["tensors"][0].__setitem__("payload_offset", data_size))
    with pytest.raises(RuntimeError, match=r"payload.*bounds"):
        SharedTensorStore.attach(ns)
    creator.close()


@pytest.mark.parametrize("layout", [
    {"shape": [2, 3], "stride": [1, 1]}, {"shape": [3, 3], "stride": [2, 2]}, {"shape": [2, 3], "stride": [4, 1]},
    {"shape": [2, 3], "stride": [3]}, {"shape": [-2, 3], "stride": [3, 1]}, {"shape": [2, 3], "stride": [3, -1]},
    {"shape": [True, 3], "stride": [3, 1]}, {"shape": [2, 3], "stride": [3, True]},
    {"shape": [2.0, 3], "stride": [3, 1]}, {"shape": None, "stride": [3, 1]}, {"shape": [2, 3], "stride": None},
])
def test_attach_rejects_invalid_layout(ns, layout):
    # test_shared_tensor_store.py:584-614
    creator = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    _rewrite_manifest(ns, lambda m: m["tensors"][0].update(layout))
    with pytest.raises(RuntimeError, match=r"manifest.*(shape|stride|layout)"):
        SharedTensorStore.attach(ns)
    creator.close()


def test_second_creator_fails_and_first_survives(ns):
    # test_shared_tensor_store.py:617-630
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    with pytest.raises(FileExistsError):
        SharedTensorStore.create_from_model(ns, src, parameter_names=["weight"])
    follower = SharedTensorStore.attach(ns)
    target = _Mixed(device="meta")
    follower.materialize_into(target, device="cpu")
    torch.testing.assert_close(target.weight, src.weight)
    follower.close()
    creator.close()
    assert not [f for f in os.listdir("/dev/shm") if f.startswith(f".{store_segment_name(ns)}.")]


def test_attach_missing_fails(ns):
    # test_shared_tensor_store.py:655-658
    with pytest.raises(FileNotFoundError):
        SharedTensorStore.attach(ns)


def test_close_is_idempotent(ns):
    # test_shared_tensor_store.py:661-668
    store = SharedTensorStore.create_from_model(ns, _Mixed(), parameter_names=["weight"])
    store.close()
    store.close()
    assert not os.path.exists(os.path.join("/dev/shm", store_segment_name(ns)))
    with pytest.raises(RuntimeError, match="closed"):
        store.materialize_into(_Mixed(device="meta"), device="cpu")


# ---- across processes ------------------------------------------------------------------


def _follower(ns: str, q) -> None:
    try:
        store = SharedTensorStore.attach(ns)
        target = _Mixed(device="meta")
        store.materialize_into(target, device="cpu")
        store.close()
        q.put((target.weight.detach().tolist(), target.counter.tolist(), float(target.scalar)))
    except BaseException as err:  # report to the parent instead of hanging it
        q.put(repr(err))


def test_follower_in_another_process(ns):
    src = _Mixed()
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=["weight", "scalar"])
    try:
        ctx = mp.get_context("spawn")
        q = ctx.Queue()
        p = ctx.Process(target=_follower, args=(ns, q))
        p.start()
        got = q.get(timeout=120)
        p.join(timeout=60)
        assert p.exitcode == 0, got
        assert got == (src.weight.detach().tolist(), src.counter.tolist(), 7.5)
    finally:
        creator.close()


# ---- a closed segment never unmaps memory that tensors still view -----------------------


def _mapped(addr: int) -> bool:
    """Whether a shared-memory mapping of this process covers ``addr``."""
    with open("/proc/self/maps") as fh:
        for line in fh:
            lo, hi = (int(x, 16) for x in line.split()[0].split("-"))
            if lo <= addr < hi and "/dev/shm/" in line:
                return True
    return False


def test_close_keeps_live_views_readable_and_unmaps_with_the_last(ns):
    """The cause of a segfault in the shared-memory streaming release: a segment closed while
    ``torch.frombuffer`` views were alive unmapped their memory. Now the views stay readable, the name is
    gone at once, and the mapping goes with the last view."""
    import gc

    seg = SharedSegment(f"{ns}_v", 1 << 20, create=True)
    path = seg.path
    t = torch.frombuffer(seg.buf, dtype=torch.uint8)
    t.copy_(torch.arange(1 << 20, dtype=torch.int64).remainder(251).to(torch.uint8))
    view = t[4096:8192].view(torch.int32)
    addr = t.data_ptr()
    seg.close()
    seg.close()  # idempotent
    assert not os.path.exists(path)  # the creator removed the name
    with pytest.raises(RuntimeError, match="closed"):
        seg.buf
    want = torch.arange(1 << 20, dtype=torch.int64).remainder(251).to(torch.uint8)
    assert torch.equal(t, want) and torch.equal(view.view(torch.uint8), want[4096:8192])  # still mapped
    assert _mapped(addr)
    del t, view
    gc.collect()
    assert not _mapped(addr)  # unmapped once the last view went


def test_close_without_views_unmaps_at_once(ns):
    seg = SharedSegment(f"{ns}_n", 1 << 16, create=True)
    seg.buf[0] = 1
    addr = torch.frombuffer(seg.buf, dtype=torch.uint8).data_ptr()  # the temporary view is gone at once
    assert _mapped(addr)
    seg.close()
    assert not _mapped(addr)


def test_release_after_shared_memory_streaming_leaves_parameters_readable(ns):
    """tensor_manager.py:2320-2354: release(preserve_model=True) copies shared-memory blocks out into the
    parameters; the block segments go, and the parameters stay readable and equal to the originals."""
    from unittest import mock

    import flextensor_amd.manager as M
    from flextensor_amd.allocation_block import HostPinner
    from flextensor_amd.controllers import AllocationBlockController
    from flextensor_amd.planner import TensorStatistics

    model = nn.Sequential(nn.Linear(64, 32), nn.Linear(32, 64))
    params = list(model.parameters())
    want = [p.detach().clone() for p in params]
    units = {"0": list(model[0].parameters()), "1": list(model[1].parameters())}
    tensors = {id(p): p for p in params}
    strategy = {x: [TensorStatistics(id(p), f"{x}.{i}", p.numel() * p.element_size(), 0.0)
                    for i, p in enumerate(ps)] for x, ps in units.items()}
    names = {x: f"{ns}_b{x}" for x in units}
    ctrl = AllocationBlockController({0: ["0"], 1: ["1"]}, torch.device("cpu"), tensors, strategy, {"0": 0, "1": 1},
                                     host_pinner=HostPinner("torch", enabled=False), shm_block_name_map=names)
    ctrl.commit_construction()
    for tid, view in ctrl.get_tensor_id_to_view_mapping().items():
        tensors[tid].data = view  # the parameters alias their slots, as when streaming
    for x in units:
        ctrl.schedule_transfer(x)
    mgr = M.OffloadManager(f"shm-release-{ns}")
    mgr.model, mgr.controller, mgr.device = model, ctrl, torch.device("cpu")
    # as in a streaming run, the loader's shutdown releases the controller's blocks (and their segments)
    # after release() took the views it restores from, and before it copies them out
    mgr.loader = type("_Loader", (), {"shutdown": staticmethod(ctrl.shutdown)})()
    mgr.units = [M._Unit(x, model[int(x)], ps, [f"{x}.w", f"{x}.b"]) for x, ps in units.items()]
    with mock.patch.object(M.torch.cuda, "synchronize", lambda *a: None):
        mgr.release()
    del ctrl
    import gc

    gc.collect()
    for p, w in zip(params, want):
        assert torch.equal(p, w)  # readable after the blocks' segments were released
    assert not [f for f in os.listdir("/dev/shm") if f.startswith(f"{ns}_b")]
