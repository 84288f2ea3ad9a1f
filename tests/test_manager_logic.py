"""CPU tests of the offload manager's host logic: unit selection, config, planning."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from flextensor_amd.config import OffloadConfig, load_config_from_env
from flextensor_amd.manager import _Unit, plain_tensors, plan_streaming, select_offload_units, shared_unit_parameters
from flextensor_amd.planner import LayerStatistics, check_overlap_constraint, check_transfer_constraint
from flextensor_amd.workloads import LlamaModel, LlamaShape


def test_select_units_llama():
    m = LlamaModel(LlamaShape(n_layers=3, hidden=16, n_heads=2, n_kv_heads=2, head_dim=8, inter=32, vocab=50,
                              max_seq=8))
    assert select_offload_units(m, ["layers.*"], []) == ["layers.0", "layers.1", "layers.2"]
    assert select_offload_units(m, ["*"], []) == ["embed", "layers.0", "layers.1", "layers.2", "norm", "lm_head"]
    assert select_offload_units(m, ["layers.*"], ["layers.1"]) == ["layers.0", "layers.2"]
    assert select_offload_units(m, ["class:DecoderLayer"], []) == ["layers.0", "layers.1", "layers.2"]
    assert select_offload_units(m, ["layers.**"], []) == ["layers.0", "layers.1", "layers.2"]
    assert select_offload_units(m, ["layers.*.attn"], []) == ["layers.0.attn", "layers.1.attn", "layers.2.attn"]


def test_config_defaults_and_env(monkeypatch):
    c = OffloadConfig()
    assert (c.num_blocks, c.min_blocks, c.pinned_memory_mode, c.transfer_mode) == (
        4, 4, "torch", "allocation_block_transfer")
    assert c.include_patterns == ["*"] and c.profiling_iters == 10 and c.discovery_iters == 1
    with pytest.raises(ValueError):
        OffloadConfig(num_blocks=1)
    with pytest.raises(ValueError):
        OffloadConfig(transfer_mode="nope")
    monkeypatch.setenv("FT_NUM_BLOCKS", "6")
    monkeypatch.setenv("FT_INCLUDE_PATTERNS", "layers.*")
    c = load_config_from_env()
    assert c.num_blocks == 6 and c.include_patterns == ["layers.*"]
    assert c.enabled is False  # from the environment alone offloading needs FT_ENABLED=1


def _mk(sizes):
    return [_Unit(f"l{i}", nn.Identity(), [nn.Parameter(torch.empty(n // 2, dtype=torch.bfloat16))])
            for i, n in enumerate(sizes)]


@pytest.mark.parametrize("n", [2, 3, 5, 8])
@pytest.mark.parametrize("blocks", [2, 3, 4])
def test_plan_all_streamed_is_hazard_free(n, blocks):
    units = _mk([1000] * n)
    order = [u.label for u in units]
    plan = plan_streaming(units, order, None, 0, blocks)
    assert plan.streamed == order and not plan.resident
    bd = plan.block_data
    stats = [LayerStatistics(x) for x in order]
    assert check_overlap_constraint(bd.transfer_to_compute_map, stats, bd.label_to_block_id)
    assert check_transfer_constraint(bd.transfer_to_compute_map, bd.label_to_block_id, stats)
    assert sorted(bd.transfer_to_compute_map.values()) == sorted(order)  # every unit fed once


def test_plan_fits_budget_and_spreads_streamed_units():
    units = _mk([1000] * 10)
    order = [u.label for u in units]
    plan = plan_streaming(units, order, budget=7000, base_bytes=500, num_blocks=2)
    assert plan.planned_gpu_bytes <= 7000
    assert plan.resident and plan.streamed and plan.reordered
    k = len(plan.streamed)
    assert 500 + (10 - k) * 1000 + sum(plan.block_data.block_sizes.values()) <= 7000
    # no fewer streamed units would fit
    assert 500 + (10 - (k - 1)) * 1000 + 2 * 1000 > 7000


@pytest.mark.parametrize("n", [4, 7, 10, 32])
def test_streamed_units_start_at_the_first_unit_and_keep_the_centred_gaps(n):
    """The streamed picks are the centred ones rotated to start at the first unit: the cyclic gaps are
    unchanged, and the first unit's transfer is a cyclic preload issued in the previous pass."""
    from flextensor_amd.loaders import find_transfers_for_preload

    units = _mk([1000] * n)
    order = [u.label for u in units]
    seen = set()
    for budget in range(2000 + 1000, 1000 * n + 1, 500):
        plan = plan_streaming(units, order, budget=budget, base_bytes=0, num_blocks=2, min_blocks=2)
        if plan.block_data is None or len(plan.streamed) in seen:
            continue
        k = len(plan.streamed)
        seen.add(k)
        idx = [order.index(x) for x in plan.streamed]
        centred = sorted({min(n - 1, int((i + 0.5) * n / k)) for i in range(k)})

        def gaps(p):
            return [b - a for a, b in zip(p, p[1:])] + [n - p[-1] + p[0]]

        assert idx[0] == 0 and gaps(idx) == gaps(centred), (k, idx, centred)
        if plan.resident:
            bd = plan.block_data
            stats = [LayerStatistics(x) for x in order]
            pre = find_transfers_for_preload(bd.transfer_to_compute_map, stats)
            assert order[0] in pre.values(), (k, bd.transfer_to_compute_map)
    assert seen


def test_plan_everything_resident_when_it_fits():
    units = _mk([100] * 4)
    plan = plan_streaming(units, [u.label for u in units], budget=10_000, base_bytes=0, num_blocks=2)
    assert plan.block_data is None and plan.streamed == []


def test_plan_rejects_impossible_budget():
    units = _mk([1000] * 4)
    with pytest.raises(RuntimeError, match="Insufficient GPU budget"):
        plan_streaming(units, [u.label for u in units], budget=1500, base_bytes=0, num_blocks=2)


def test_copy_policy_from_measured_curves():
    """The link sweep measured on the MI355X picks the kernel only for chunks up to 1 MiB."""
    from flextensor_amd.link_model import CopyCurve, choose_copy_policy

    gbps = {  # bench.py --link-sweep on the MI355X (GB/s per size)
        "sdma": {65536: 5.06, 262144: 14.66, 1048576: 33.74, 2097152: 42.56, 4194304: 48.57, 16777216: 54.88,
                 67108864: 56.67, 188743680: 57.09, 536870912: 57.24},
        "kernel": {65536: 10.12, 262144: 25.8, 1048576: 43.62, 2097152: 43.33, 4194304: 49.96, 16777216: 55.24,
                   67108864: 56.69, 188743680: 57.04, 536870912: 57.14},
        "sdma_split2": {65536: 1.77, 262144: 4.35, 1048576: 19.76, 2097152: 28.45, 4194304: 38.51,
                        16777216: 50.05, 67108864: 55.2, 188743680: 56.57, 536870912: 56.92},
    }
    curves = {e: CopyCurve(e, {n: n / (g * 1e9) * 1e3 for n, g in t.items()}) for e, t in gbps.items()}
    kmax, split_min, n_streams = choose_copy_policy(curves["sdma"], curves["kernel"], curves["sdma_split2"], 2)
    assert kmax == 1 << 20  # 2 MiB is only 2% faster on the kernel: not worth its cost to kernels beside it
    assert split_min == 2**63 - 1 and n_streams == 1  # splitting never helps
    assert choose_copy_policy(curves["sdma"], curves["kernel"], min_kernel_gain=1.0)[0] == 64 << 20


def test_block_range_is_validated():
    """config.py:468-472: num_blocks below min_blocks is refused."""
    with pytest.raises(ValueError, match="must be >= min_blocks"):
        OffloadConfig(num_blocks=2)  # min_blocks defaults to 4
    assert OffloadConfig(num_blocks=2, min_blocks=2).num_blocks == 2


def test_slot_count_is_the_largest_in_range_that_fits():
    """Fewest streamed units first; then the deepest ring in [min_blocks, num_blocks] within the budget."""
    units = _mk([1000] * 12)
    order = [u.label for u in units]
    roomy = plan_streaming(units, order, budget=10_500, base_bytes=0, num_blocks=4, min_blocks=2)
    tight = plan_streaming(units, order, budget=10_500, base_bytes=0, num_blocks=2, min_blocks=2)
    assert len(roomy.streamed) == len(tight.streamed)  # the slot count never costs a resident unit
    assert len(roomy.block_data.block_sizes) >= len(tight.block_data.block_sizes)
    assert roomy.planned_gpu_bytes <= 10_500 and tight.planned_gpu_bytes <= 10_500
    fixed = plan_streaming(units, order, budget=10_500, base_bytes=0, num_blocks=4)  # min_blocks = num_blocks
    # 8 resident units + 2 slots fit 10_500; with the range pinned at 4 slots only 6 units stay resident
    assert (len(roomy.streamed), len(roomy.block_data.block_sizes)) == (4, 2)
    assert (len(fixed.streamed), len(fixed.block_data.block_sizes)) == (6, 4)
    # with equal units a slot costs what keeping one more unit resident costs, so slack keeps units resident
    cheaper = plan_streaming(units, order, budget=11_000, base_bytes=0, num_blocks=4, min_blocks=2)
    assert (len(cheaper.streamed), len(cheaper.block_data.block_sizes)) == (3, 2)
    deeper = plan_streaming(units, order, budget=None, base_bytes=0, num_blocks=4, min_blocks=2)
    assert len(deeper.streamed) == 12 and len(deeper.block_data.block_sizes) == 4  # no budget: the deepest ring
    for p in (roomy, tight, fixed, cheaper, deeper):
        stats = [LayerStatistics(x) for x in order]
        assert check_overlap_constraint(p.block_data.transfer_to_compute_map, stats, p.block_data.label_to_block_id)


def test_plan_budget_exhausted_by_outside_tensors_names_the_reservation():
    """gpu_budget.py:200-225: when the tensors kept on the GPU outside the units leave no room for the
    ring, planning fails with a RuntimeError that states the budget, the reservation and the minimum."""
    units = _mk([1000] * 6)
    order = [u.label for u in units]
    plan = plan_streaming(units, order, budget=2000 + 500, base_bytes=500, num_blocks=2)  # just fits
    assert plan.streamed == order
    with pytest.raises(RuntimeError, match=r"budget=2499 bytes, reserved_outside_units=500 bytes, "
                                           r"effective_budget=1999 bytes, minimum_ring=2000 bytes"):
        plan_streaming(units, order, budget=2499, base_bytes=500, num_blocks=2)


def test_plain_tensors_reaches_attributes_and_containers_once():
    """The tensors outside parameters and buffers that go to the GPU with the rest of the model: plain
    attributes, tensors in lists, tuples, dicts and plain objects, each once (the reference's unmapped
    tensors, tensor_processors.py:324-360,685-742; its reachable-tensor cases in
    tests/unit/test_tensor_processors.py:293-356,513-553)."""

    class Holder:
        pass

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.lin = nn.Linear(4, 4)
            self.register_buffer("b", torch.zeros(3))
            self.plain = torch.ones(2)
            self.alias = self.plain
            self.lst = [torch.ones(5), (torch.ones(6), {"k": torch.ones(7)})]
            self.lst.append(self.lst)  # a list that holds itself
            h = Holder()
            h.t, h.me = torch.ones(8), h
            self.holder = h
            self.tied = self.lin.weight  # a parameter: placed with the parameters
            self.buf_ref = [self.b]  # a buffer: placed with the buffers
            self.namespace = torch  # a Python module is not entered
            self.child = nn.Sequential(nn.Linear(2, 2))

    m = M()
    m.child.extra = torch.ones(9)  # a plain attribute of a submodule
    got = plain_tensors(m)
    assert [tuple(t.shape) for t in got] == [(2,), (5,), (6,), (7,), (8,), (9,)]
    assert got[0] is m.plain and got[4] is m.holder.t
    registered = {id(t) for t in m.parameters()} | {id(t) for t in m.buffers()}
    assert not any(id(t) in registered for t in got)


def test_parameters_held_by_two_units_are_found():
    """Tied weights (one Parameter registered in two units' modules) are reported with every unit holding
    them; a module reused under one name is not a tie."""
    m = nn.Module()
    m.layers = nn.ModuleList(nn.Linear(4, 4) for _ in range(4))
    m.layers[3].weight = m.layers[0].weight
    m.layers[2].bias = m.layers[1].bias
    labels = [f"layers.{i}" for i in range(4)]
    got = shared_unit_parameters(m, labels)
    assert got == {id(m.layers[0].weight): ["layers.0", "layers.3"], id(m.layers[1].bias): ["layers.1", "layers.2"]}
    assert shared_unit_parameters(m, ["layers.0", "layers.1"]) == {}
    n = nn.Module()
    block = nn.Linear(4, 4)
    n.a, n.b = block, nn.Linear(4, 4)
    assert shared_unit_parameters(n, ["a", "b"]) == {}
