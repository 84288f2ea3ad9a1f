"""Units kept exponent-coded in HBM (``encode_resident_blocks``), on the CPU: which resident units the
planner encodes, that the budget counts the encoded blocks and their shared decode slot, that a restored
plan encodes the same units, and that a block's encoded size is known before it is packed for real."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from flextensor_amd import expcode
from flextensor_amd.config import OffloadConfig
from flextensor_amd.layout import pack_into, plan_block
from flextensor_amd.manager import _Unit, encode_residents, plan_from_state, plan_streaming, state_from_plan
from oracle import expcode as X


def _mk(sizes):
    return [_Unit(f"l{i}", nn.Identity(), [nn.Parameter(torch.empty(n // 2, dtype=torch.bfloat16))],
                  [f"l{i}.w"]) for i, n in enumerate(sizes)]


def test_encode_residents_takes_the_fewest_and_counts_one_slot():
    raw = {x: 1000 for x in "abcd"}
    enc = {"a": (600, 1000), "b": (500, 1000), "c": (600, 1000), "d": (600, 1000)}
    assert encode_residents(list("abcd"), raw, enc, 4000) == ({}, 4000)  # fits raw: nothing encoded
    # b saves most, then a, c, d (ties in pass order); the 1000-byte decode slot is counted once:
    # b: 3500 + 1000 = 4500, +a: 4100, +c: 3700, +d: 3300
    assert encode_residents(list("abcd"), raw, enc, 3999) == ({"b": 500, "a": 600, "c": 600}, 3700)
    assert encode_residents(list("abcd"), raw, enc, 3699) == ({"b": 500, "a": 600, "c": 600, "d": 600}, 3300)
    assert encode_residents(list("abcd"), raw, enc, 3299) is None
    # the slot is the largest packed raw block among the encoded units: e saves 2000 bytes, but its
    # 3008-byte slot leaves 2000 + 3008 (e) and 1600 + 3008 (e, a), above the raw 4000
    assert encode_residents(["a", "e"], {"a": 1000, "e": 3000}, {"a": (600, 1000), "e": (1000, 3008)},
                            3999) is None
    # a unit that does not shrink is never a candidate
    assert encode_residents(["a"], {"a": 1000}, {"a": (1000, 1000)}, 999) is None


def test_plan_streams_fewer_units_with_encoded_residents():
    units = _mk([1000] * 12)
    order = [u.label for u in units]
    encodable = {x: (752, 1000) for x in order}
    budget = 9000
    raw_plan = plan_streaming(units, order, budget, 500, 2)
    plan = plan_streaming(units, order, budget, 500, 2, encodable=encodable)
    assert not raw_plan.encoded_resident
    assert len(plan.streamed) < len(raw_plan.streamed)
    ring = sum(plan.block_data.block_sizes.values())
    n_enc = len(plan.encoded_resident)
    assert n_enc and set(plan.encoded_resident) <= set(plan.resident)
    assert all(v == 752 for v in plan.encoded_resident.values())
    want = 500 + ring + 1000 + 752 * n_enc + 1000 * (len(plan.resident) - n_enc)
    assert plan.planned_gpu_bytes == want <= budget
    # one more unit streamed than needed would not have been chosen: one fewer does not fit
    k = len(plan.streamed)
    assert 500 + ring + 1000 + 752 * (12 - k + 1) > budget
    # everything fits raw: no encoding even when allowed
    roomy = plan_streaming(units, order, 20_000, 0, 2, encodable=encodable)
    assert not roomy.streamed and not roomy.encoded_resident


def test_restored_plan_encodes_the_same_units():
    units = _mk([1000] * 12)
    order = [u.label for u in units]
    encodable = {x: (752, 1000) for x in order}
    plan = plan_streaming(units, order, 9000, 0, 2, encodable=encodable)
    model = nn.ParameterList([p for u in units for p in u.params])
    st = state_from_plan(model, units, plan, {}, "allocation_block_transfer")
    again = plan_from_state(st, units, 0, 9000, encodable)
    assert again.streamed == plan.streamed and again.encoded_resident == plan.encoded_resident
    assert again.planned_gpu_bytes == plan.planned_gpu_bytes
    assert not plan_from_state(st, units, 0, 9000).encoded_resident  # without the option: raw residents


def test_pack_into_zeroes_the_gaps():
    ts = [torch.arange(5, dtype=torch.int16), torch.arange(3, dtype=torch.bfloat16)]
    slots, total = plan_block(ts, 128)
    block = torch.full((total,), 0xEE, dtype=torch.uint8)
    pack_into(block, slots, ts)
    covered = torch.zeros(total, dtype=torch.bool)
    for s in slots:
        covered[s.offset: s.offset + s.nbytes] = True
    assert total == 128 + 128 and not block[~covered].any()


def test_packed_encoded_size_is_exact():
    g = torch.Generator().manual_seed(5)
    ts = [(torch.randn(n, generator=g) * 0.02).to(torch.bfloat16) for n in (3000, 777, 4096)]
    ts.append(torch.randn(40, 30, generator=g).to(torch.bfloat16).t())  # not dense in row order: packed as is
    ts.append(torch.randn(64, generator=g).to(torch.bfloat16)[::2])  # gaps: packed element-wise
    size, raw = expcode.packed_encoded_size(ts, 128)
    slots, total = plan_block(ts, 128)
    block = torch.full((total,), 0x5A, dtype=torch.uint8)
    pack_into(block, slots, ts)
    assert raw == total
    assert size == X.encoded_size(block.numpy()) == X.encode(block.numpy()).size
    scratch = torch.full((total + 100,), 0x33, dtype=torch.uint8)  # a larger, dirty scratch gives the same
    assert expcode.packed_encoded_size(ts, 128, scratch) == (size, raw)
    from oracle import expcode_dense as D

    dense, _ = expcode.packed_encoded_size(ts, 128, scratch, dense=True)  # the format units kept in HBM use
    assert dense == D.encoded_size(block.numpy()) == D.encode(block.numpy()).size < size


def test_config_rules():
    assert OffloadConfig(encode_resident_blocks=True).encode_resident_blocks
    with pytest.raises(ValueError, match="encode_resident_blocks"):
        OffloadConfig(encode_resident_blocks=True, transfer_mode="raw_block_transfer")
    with pytest.raises(ValueError, match="encode_resident_blocks"):
        OffloadConfig(encode_resident_blocks=True, shm_enabled=True, shm_namespace="x")


def test_encoded_plan_streams_the_fewest_bytes_of_unequal_units():
    """Attention units of 1342 bytes and MLP projections of 902 (the 7B-shape decoder's finer units,
    scaled down 10^5): the fewest streamed units that fit (32, every attention unit) are not the fewest
    streamed bytes (36 units, more of them small)."""
    sizes = [1342, 902, 902, 902] * 32
    units = _mk(sizes)
    order = [u.label for u in units]
    encodable = {u.label: (int(u.nbytes * 0.7523) + u.nbytes // 1024, u.nbytes) for u in units}
    budget, base = 80_000, 5_243
    plan = plan_streaming(units, order, budget, base, 2, 2, encodable)
    by = {u.label: u.nbytes for u in units}
    got = sum(by[x] for x in plan.streamed)
    assert plan.planned_gpu_bytes <= budget
    # every count from 1 up: the first that fits streams more bytes than the plan chosen
    first = None
    for k in range(1, len(units) + 1):
        centred = sorted({min(len(units) - 1, int((i + 0.5) * len(units) / k)) for i in range(k)})
        picked = [order[i - centred[0]] for i in centred]
        resident = [x for x in order if x not in picked]
        if encode_residents(resident, by, encodable, budget - base - 2 * 1342) is not None:
            first = sum(by[x] for x in picked)
            break
    assert first is not None and got < first
    assert len(plan.streamed) > 32
    raw = plan_streaming(units, order, budget, base, 2, 2)  # without encoding: the reference's fewest units
    assert not raw.encoded_resident
