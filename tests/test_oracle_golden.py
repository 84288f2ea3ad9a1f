"""Pins the oracle: every oracle function against the reference's own fixtures,
closed forms and properties chosen so that a plausible slip fails a check."""

from __future__ import annotations

import json
import math
import random
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import interpolator as oi
from oracle import layout as ol
from oracle import native as onat
from oracle import planner as op
from oracle import schedule as osch

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_cases.json").read_text())


def _intkeys(d):
    return {int(k): v for k, v in d.items()}


# ---- planner ---------------------------------------------------------------


@pytest.mark.parametrize("n,expected", GOLD["min_blocks_sequential"]["cases"])
def test_min_blocks_table(n, expected):
    assert op.min_blocks_sequential([f"layer_{i}" for i in range(n)]) == expected


def test_min_block_sizes_docstring_example():
    c = GOLD["min_block_sizes"]
    assert op.block_sizes(c["sizes"], _intkeys(c["allocation"])) == _intkeys(c["expected"])


def test_single_layer_distribution():
    c = GOLD["single_layer_distribution"]
    assert op.optimize_block_distribution([x for x, _ in c["sizes"]], c["num_blocks"]) == _intkeys(c["expected"])
    assert op.find_minimum_blocks([]) == (0, {})


@pytest.mark.parametrize("n", [2, 3, 5, 8, 17])
@pytest.mark.parametrize("blocks", [2, 3, 4])
def test_distribution_properties(n, blocks):
    labels = [f"layer_{i}" for i in range(n)]
    alloc = op.optimize_block_distribution(labels, blocks)
    owner = {x: b for b, xs in alloc.items() for x in xs}
    assert sorted(owner) == sorted(labels)
    assert all(owner[a] != owner[b] for a, b in zip(labels, labels[1:]))  # neighbours never share
    counts = sorted(len(v) for v in alloc.values())
    assert counts[-1] - counts[0] <= 1  # load balanced
    assert owner[labels[0]] == 0 and owner[labels[1]] == 1  # lowest free slot first


def test_distribution_rejects_too_few_blocks():
    with pytest.raises(ValueError, match="at least 2"):
        op.optimize_block_distribution(["a", "b"], 1)


def test_allocate_with_capacity_backtracks():
    # sizes force label c away from slot 0 although colouring alone would allow it
    sizes = [("a", 6), ("b", 6), ("c", 5), ("d", 1)]
    alloc = op.allocate_blocks(sizes, 3, capacity=10)
    assert alloc == {0: ["a", "d"], 1: ["b"], 2: ["c"]}
    n, alloc2 = op.find_minimum_blocks(sizes, capacity=10)
    assert n == 3 and alloc2 == alloc
    assert op.find_minimum_blocks(sizes)[0] == 2


@pytest.mark.parametrize("case", GOLD["find_transfers_for_preload"]["cases"], ids=lambda c: c["name"])
def test_preload_examples(case):
    assert op.find_transfers_for_preload(case["t2c"], GOLD["find_transfers_for_preload"]["layers"]) == case["expected"]


def test_preload_empty():
    for t2c, layers in GOLD["find_transfers_for_preload"]["empty_cases"]:
        assert op.find_transfers_for_preload(t2c, layers) == {}


@pytest.mark.parametrize("case", GOLD["create_allocation_ordered"]["cases"], ids=lambda c: c["name"])
def test_allocation_ordered_examples(case):
    out = op.create_allocation_ordered(case["l2b"], case["layers"])
    assert out == _intkeys(case["expected"])


@pytest.mark.parametrize("case", GOLD["rearrange_transfers_empty"]["cases"])
def test_rearrange_empty_inputs(case):
    assert list(op.rearrange_transfers(case["t2c"], case["l2b"], case["layers"])) == case["expected"]


def _chain_schedule(labels, gaps, blocks=2):
    offloaded = [x for x in labels if x not in gaps]
    t2c = {offloaded[i]: offloaded[i + 1] for i in range(len(offloaded) - 1)}
    l2b = {offloaded[i]: i % blocks for i in range(len(offloaded) - 1)}
    return t2c, l2b


def test_rearrange_moves_into_gap_and_keeps_constraints():
    labels = ["embed", "L0", "L1", "L2", "L3", "L4"]
    t2c, l2b = _chain_schedule(labels, {"L2"})
    new_t2c, new_l2b, remapped = op.rearrange_transfers(t2c, l2b, labels)
    assert op.check_transfer_constraint(new_t2c, new_l2b, labels)
    assert op.check_overlap_constraint(new_t2c, labels, new_l2b)
    assert sorted(new_t2c.values()) == sorted(t2c.values())  # every consumer still fed once
    # the transfer feeding L3 may now start in the gap label L2 or earlier
    moved = {c: t for t, c in new_t2c.items()}
    assert labels.index(moved["L3"]) <= labels.index("L2")


def test_rearrange_identity_when_no_gap():
    labels = ["a", "b", "c"]
    t2c, l2b = {"a": "b"}, {"a": 0}
    new_t2c, new_l2b, remapped = op.rearrange_transfers(t2c, l2b, labels)
    assert new_t2c == {"a": "b"} and new_l2b == {"a": 0} and remapped == {"a": "a"}


def test_overlap_constraint_detects_shared_position():
    # same slot: transfer at position 1 while a compute of that slot is at 1
    assert not op.check_overlap_constraint({"a": "b", "b": "c"}, ["a", "b", "c"], {"a": 0, "b": 0})
    assert op.check_overlap_constraint({"a": "b", "b": "c"}, ["a", "b", "c"], {"a": 0, "b": 1})


def test_prepare_block_strategy_chain():
    layers = ["l0", "l1", "l2", "l3"]
    layer_tensors = {x: [i] for i, x in enumerate(layers)}
    # tensors of label l(i+1) are transferred at l(i); l0's at l3 (cyclic)
    strategy = {"l0": [(1, 100)], "l1": [(2, 300)], "l2": [(3, 200)], "l3": [(0, 50)]}
    out = op.prepare_block_strategy(layers, layer_tensors, strategy, 2)
    assert out["transfer_to_compute_map"] == {"l0": "l1", "l1": "l2", "l2": "l3", "l3": "l0"}
    assert out["allocation_ordered"] == {0: ["l0", "l2"], 1: ["l1", "l3"]}
    assert out["block_sizes"] == {0: 200, 1: 300}
    assert op.find_transfers_for_preload(out["transfer_to_compute_map"], layers) == {"l3": "l0"}


# ---- schedule traces -------------------------------------------------------


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_oracle_reproduces_frozen_trace(kind):
    c = GOLD["frozen_trace"]
    log = osch.trace(kind, c["labels"], c["transfer_to_compute_map"], c["label_to_block_id"], osch.passes(c["labels"]))
    assert [[o, s] for o, s, _ in log] == c["expected"][kind]


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_oracle_trace_invariants(kind):
    labels = ["embed", "L0", "L1", "L2", "L3"]
    t2c, l2b = _chain_schedule(labels, set())
    log = osch.trace(kind, labels, t2c, l2b, osch.passes(labels, 2))
    # every consumer waits (on compute) for its transfer before its forward
    for t, c in t2c.items():
        sched = [i for i, e in enumerate(log) if e[0] == "schedule_transfer" and e[2] == t]
        fwd = [i for i, e in enumerate(log) if e[0] == "forward" and e[2] == c]
        for s, f in zip(sched, fwd[:: 1]):
            pass
        ev = {e[2]: i for i, e in enumerate(log) if e[0] == "record_event" and e[1] == "transfer"}
        for s in sched:
            done = next(e[2] for e in log[s:] if e[0] == "record_event" and e[1] == "transfer")
            waits = [i for i, e in enumerate(log) if e[0] == "wait_event" and e[1] == "compute" and e[2] == done]
            assert waits, (t, c)
            later_fwd = [f for f in fwd if f > ev[done]]
            assert later_fwd and waits[0] < later_fwd[0]


# ---- layout ------------------------------------------------------------------


def test_packed_layout_known_answers():
    # 8-layer MLP layer at 4096 -> 11008 -> 4096 in bf16 with biases
    sizes = [11008 * 4096 * 2, 11008 * 2, 4096 * 11008 * 2, 4096 * 2]
    assert ol.packed_layout(sizes) == ([0, 90177536, 90199552, 180377088], 180385280)
    assert onat.packed_layout(sizes) == ol.packed_layout(sizes)
    assert ol.packed_layout([]) == ([], 0)
    assert ol.packed_layout([1, 1, 1]) == ([0, 128, 256], 384)
    assert ol.raw_layout([3, 5, 7]) == ([0, 3, 8], 15)


@pytest.mark.parametrize("bad", GOLD["alignment_rejects"]["values"])
def test_packed_layout_rejects_bad_alignment(bad):
    with pytest.raises(ValueError, match="positive integer"):
        ol.packed_layout([1], bad)


def test_packed_layout_properties():
    rng = random.Random(5)
    for _ in range(200):
        sizes = [rng.choice([0, 1, 2, 127, 128, 129, rng.randrange(1, 1 << 20)]) for _ in range(rng.randrange(1, 20))]
        a = rng.choice([1, 2, 16, 128, 256])
        offs, total = ol.packed_layout(sizes, a)
        assert all(o % a == 0 for o in offs) and total % a == 0
        ends = [o + s for o, s in zip(offs, sizes)]
        assert all(e <= nxt for e, nxt in zip(ends, offs[1:] + [total]))  # no overlap, fits
        assert all(nxt - e < a for e, nxt in zip(ends, offs[1:] + [total]))  # minimal padding
        assert onat.packed_layout(sizes, a) == (offs, total)


def test_dense_layout_cases():
    s = GOLD["strides"]
    assert ol.is_dense(tuple(s["fortran_4x3"]["shape"]), tuple(s["fortran_4x3"]["stride"]))
    nd = s["non_dense"]
    assert not ol.is_dense(tuple(nd["shape"]), tuple(nd["stride_in"]))
    assert ol.packed_strides(tuple(nd["shape"]), tuple(nd["stride_in"])) == tuple(nd["stride_packed"])
    assert ol.is_dense((), ())
    assert ol.is_dense((0,), (1,))
    assert ol.is_dense((4, 2, 3), (1, 12, 4))  # permuted 3-D
    assert not ol.is_dense((3, 2, 5), (20, 10, 1))  # sliced 3-D
    assert not ol.is_dense((4,), (3,))


# ---- block pack -----------------------------------------------------------------

_NP = {"float32": np.float32, "int32": np.int32}


def _pack_fixture():
    c = GOLD["allocation_block_pack"]
    return c, [np.full(t["numel"], t["fill"], dtype=_NP[t["dtype"]]) for t in c["tensors"]]


def _expected_block(c) -> bytes:
    """The fixture's block written out with ``struct``, independently of the oracle."""
    out = bytearray(c["total"])
    for t, off in zip(c["tensors"], c["offsets"]):
        raw = struct.pack("<%d%s" % (t["numel"], "f" if t["dtype"] == "float32" else "i"), *([t["fill"]] * t["numel"]))
        out[off: off + len(raw)] = raw
    return bytes(out)


def test_pack_known_answer():
    c, srcs = _pack_fixture()
    offs, total = ol.packed_layout([s.nbytes for s in srcs], c["alignment"])
    assert (offs, total) == (c["offsets"], c["total"])
    block = np.zeros(total, np.uint8)
    onat.pack(block, offs, srcs)
    assert block.tobytes() == _expected_block(c)
    # 1.0f, 2.0f and int32 3 spelled out byte by byte, little-endian
    assert block[0:4].tobytes() == b"\x00\x00\x80\x3f" and block[128:132].tobytes() == b"\x00\x00\x00\x40"
    assert block[256:260].tobytes() == b"\x03\x00\x00\x00" and not block[308:].any() and not block[48:128].any()


@pytest.mark.parametrize("wrong", [[0, 124, 256], [0, 128, 252], [4, 128, 256], [0, 256, 128]])
def test_pack_known_answer_catches_a_wrong_offset(wrong):
    c, srcs = _pack_fixture()
    block = np.zeros(c["total"], np.uint8)
    onat.pack(block, wrong, srcs)
    assert block.tobytes() != _expected_block(c)


def test_pack_keeps_fortran_memory_order():
    import torch

    f = GOLD["allocation_block_pack"]["fortran"]
    t = torch.arange(12, dtype=torch.float32).reshape(*f["base_shape"]).t()
    assert tuple(t.shape) == tuple(f["shape"]) and t.stride() == tuple(f["stride"])
    raw = np.frombuffer(bytes(t.untyped_storage()), dtype=np.uint8)
    block = np.zeros(128, np.uint8)
    onat.pack(block, [0], [raw])
    assert block[:48].tobytes() == struct.pack("<12f", *f["memory_order_values"])
    assert t.contiguous().numpy().tobytes() != block[:48].tobytes()  # a pack in C order would fail the check


def test_pack_rejects_overruns():
    with pytest.raises(ValueError, match="overruns"):
        onat.pack(np.zeros(64, np.uint8), [32], [np.zeros(40, np.uint8)])


# ---- interpolator --------------------------------------------------------------


def _pts(d):
    return {int(k): v for k, v in d.items()}


def test_interpolator_reference_checks():
    c = GOLD["interpolator"]
    pts = _pts(c["standard"])
    for chk in c["checks"]:
        fn = oi.bytes_to_duration if chk["fn"] == "bytes_to_duration" else oi.duration_to_bytes
        v = fn(pts, chk["x"])
        if "expect_abs" in chk:
            assert abs(v - chk["expect_abs"][0]) < chk["expect_abs"][1]
        if "expect_open" in chk:
            assert chk["expect_open"][0] < v < chk["expect_open"][1]
        if "expect_below" in chk:
            assert v < chk["expect_below"]
        if "expect_above" in chk:
            assert v > chk["expect_above"]
    sp = c["single_point"]
    for x, y in sp["bytes_to_duration"]:
        assert oi.bytes_to_duration(_pts(sp["points"]), x) == y
    for x, y in sp["duration_to_bytes"]:
        assert oi.duration_to_bytes(_pts(sp["points"]), x) == y
    for b in c["bandwidth"]:
        assert abs(oi.bandwidth_mbps(_pts(b["points"])) - b["mbps"]) < 1.0
    rt = c["round_trip"]
    back = oi.duration_to_bytes(pts, oi.bytes_to_duration(pts, rt["bytes"]))
    assert abs(back - rt["bytes"]) / rt["bytes"] < rt["rel_tol"]
    back = oi.bytes_to_duration(pts, oi.duration_to_bytes(pts, rt["duration"]))
    assert abs(back - rt["duration"]) / rt["duration"] < rt["rel_tol"]


def test_interpolator_closed_forms():
    # a power law t = k * b^p is reproduced exactly in log-log space, inside and outside the range
    k, p = 3e-6, 0.9
    pts = {b: k * b**p for b in (1 << 10, 1 << 16, 1 << 24)}
    for b in (100, 5000, 1 << 20, 1 << 30):
        assert math.isclose(oi.bytes_to_duration(pts, b), k * b**p, rel_tol=1e-9)
        assert math.isclose(oi.duration_to_bytes(pts, k * b**p), b, rel_tol=1e-9)
    with pytest.raises(ValueError, match="positive"):
        oi.bytes_to_duration(pts, 0)
    with pytest.raises(ValueError, match="positive"):
        oi.duration_to_bytes(pts, -1.0)


# ---- checksum -------------------------------------------------------------------


def test_checksum_sensitivity():
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, size=3 * 4096 + 77, dtype=np.uint8)
    base = onat.checksum64(data)
    assert onat.checksum64(data.copy()) == base
    for pos in (0, 1, 4095, 4096, 8191, data.size - 1):
        flipped = data.copy()
        flipped[pos] ^= 1
        assert onat.checksum64(flipped) != base
    swapped = data.copy()  # swap two 8-byte words in different lanes and blocks
    swapped[0:8], swapped[4096:4104] = data[4096:4104].copy(), data[0:8].copy()
    assert onat.checksum64(swapped) != base
    assert onat.checksum64(np.concatenate([data, np.zeros(1, np.uint8)])) != base  # length counts
    assert onat.checksum64(np.zeros(0, np.uint8)) != onat.checksum64(np.zeros(1, np.uint8))


def test_scatter_oracle_is_memcpy():
    rng = np.random.default_rng(1)
    chunk = rng.integers(0, 256, size=10000, dtype=np.uint8)
    dsts = [np.zeros(n, np.uint8) for n in (10, 0, 999, 5000)]
    descs = [(0, 10), (10, 0), (128, 999), (5000, 5000)]
    onat.scatter(chunk, descs, dsts)
    for (off, n), d in zip(descs, dsts):
        assert np.array_equal(d, chunk[off: off + n])
