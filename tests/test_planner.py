"""Product planner == reference fixtures and == oracle on seeded random inputs."""

from __future__ import annotations

import json
import random
from collections import OrderedDict
from pathlib import Path

import pytest

from flextensor_amd import planner as P
from oracle import planner as op

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_cases.json").read_text())


def _ik(d):
    return {int(k): v for k, v in d.items()}


def _stats(labels):
    return [P.LayerStatistics(label=x) for x in labels]


@pytest.mark.parametrize("n,expected", GOLD["min_blocks_sequential"]["cases"])
def test_min_blocks(n, expected):
    planner = P.MemoryBlockPlanner(OrderedDict((f"layer_{i}", 1024) for i in range(n)))
    assert planner.find_minimum_blocks_sequential() == expected


def test_path_graph_has_no_wraparound_edge():
    g = P.MemoryBlockPlanner(OrderedDict((f"layer_{i}", 1) for i in range(5))).adjacency_graph
    assert "layer_0" not in g["layer_4"] and "layer_4" not in g["layer_0"]
    assert all(f"layer_{i + 1}" in g[f"layer_{i}"] for i in range(4))
    assert P.MemoryBlockPlanner(OrderedDict()).adjacency_graph == {}


def test_min_block_sizes_example():
    c = GOLD["min_block_sizes"]
    planner = P.MemoryBlockPlanner(OrderedDict(c["sizes"]))
    assert planner.find_minimum_block_sizes(_ik(c["allocation"])) == _ik(c["expected"])


def test_empty_and_single():
    assert P.MemoryBlockPlanner(OrderedDict()).find_minimum_blocks() == (0, {})
    c = GOLD["single_layer_distribution"]
    assert P.MemoryBlockPlanner(OrderedDict(c["sizes"])).optimize_block_distribution(1) == _ik(c["expected"])


@pytest.mark.parametrize("case", GOLD["find_transfers_for_preload"]["cases"], ids=lambda c: c["name"])
def test_preload(case):
    layers = _stats(GOLD["find_transfers_for_preload"]["layers"])
    assert P.find_transfers_for_preload(case["t2c"], layers) == case["expected"]


@pytest.mark.parametrize("case", GOLD["create_allocation_ordered"]["cases"], ids=lambda c: c["name"])
def test_allocation_ordered(case):
    assert P.create_allocation_ordered(case["l2b"], _stats(case["layers"])) == _ik(case["expected"])


@pytest.mark.parametrize("case", GOLD["rearrange_transfers_empty"]["cases"])
def test_rearrange_empty(case):
    out = P.rearrange_transfers(case["t2c"], case["l2b"], _stats(case["layers"]))
    assert list(out) == case["expected"]
    assert out[0] is not case["t2c"] and out[1] is not case["l2b"]


def _random_sizes(rng, n):
    return [(f"L{i}", rng.choice([1, 7, 64, 100, 4096, rng.randrange(1, 10**6)])) for i in range(n)]


@pytest.mark.parametrize("seed", range(40))
def test_planner_matches_oracle(seed):
    rng = random.Random(seed)
    sizes = _random_sizes(rng, rng.randrange(0, 14))
    labels = [x for x, _ in sizes]
    planner = P.MemoryBlockPlanner(OrderedDict(sizes))
    assert planner.find_minimum_blocks_sequential() == op.min_blocks_sequential(labels)
    for blocks in (1, 2, 3, 5):
        try:
            want = op.optimize_block_distribution(labels, blocks)
        except ValueError:
            with pytest.raises(ValueError):
                planner.optimize_block_distribution(blocks)
            continue
        got = planner.optimize_block_distribution(blocks)
        assert got == want and list(got) == list(want)
        assert planner.find_minimum_block_sizes(got) == op.block_sizes(sizes, want)
    cap = rng.choice([None, max([s for _, s in sizes] or [1]) * 2, max([s for _, s in sizes] or [1]) + 1])
    try:
        want = op.find_minimum_blocks(sizes, cap)
    except ValueError:
        with pytest.raises(ValueError):
            planner.find_minimum_blocks(cap)
    else:
        assert planner.find_minimum_blocks(cap) == want


def _random_schedule(rng):
    n = rng.randrange(3, 16)
    labels = [f"layer.{i}" for i in range(n)]
    gaps = set(rng.sample(labels[1:], rng.randrange(0, max(1, n // 3))))
    offloaded = [x for x in labels if x not in gaps]
    blocks = rng.choice([2, 3, 4])
    t2c = {offloaded[i]: offloaded[i + 1] for i in range(len(offloaded) - 1)}
    if rng.random() < 0.5 and len(offloaded) > 2:
        t2c[offloaded[-1]] = offloaded[0]  # cyclic transfer for the next pass
    l2b = {t: i % blocks for i, t in enumerate(t2c)}
    return labels, t2c, l2b


@pytest.mark.parametrize("seed", range(60))
def test_schedule_ops_match_oracle(seed):
    rng = random.Random(1000 + seed)
    labels, t2c, l2b = _random_schedule(rng)
    stats = _stats(labels)
    assert P.find_transfers_for_preload(t2c, stats) == op.find_transfers_for_preload(t2c, labels)
    assert P.create_allocation_ordered(l2b, stats) == op.create_allocation_ordered(l2b, labels)
    assert P.check_transfer_constraint(t2c, l2b, stats) == op.check_transfer_constraint(t2c, l2b, labels)
    assert P.check_overlap_constraint(t2c, stats, l2b) == op.check_overlap_constraint(t2c, labels, l2b)
    try:
        want = op.rearrange_transfers(t2c, l2b, labels)
    except ValueError as e:
        with pytest.raises(ValueError, match=str(e)[:20]):
            P.rearrange_transfers(t2c, l2b, stats)
        return
    got = P.rearrange_transfers(t2c, l2b, stats)
    assert got == want
    assert [list(d) for d in got] == [list(d) for d in want]  # same insertion order


@pytest.mark.parametrize("seed", range(20))
def test_prepare_block_strategy_matches_oracle(seed):
    rng = random.Random(seed)
    n = rng.randrange(2, 10)
    labels = [f"l{i}" for i in range(n)]
    layer_tensors = {x: [i * 10 + j for j in range(rng.randrange(1, 4))] for i, x in enumerate(labels)}
    strategy = {}
    for i, x in enumerate(labels):
        nxt = labels[(i + 1) % n]
        if rng.random() < 0.8:
            strategy[x] = [(tid, rng.randrange(1, 5000)) for tid in layer_tensors[nxt]]
    stats = [P.LayerStatistics(x, [P.TensorStatistics(t, str(t), 1) for t in layer_tensors[x]]) for x in labels]
    pstrat = {x: [P.TensorStatistics(t, str(t), s) for t, s in ts] for x, ts in strategy.items()}
    for blocks in (None, 2, 3):
        try:
            want = op.prepare_block_strategy(labels, layer_tensors, strategy, blocks)
        except ValueError:
            with pytest.raises(ValueError):
                P.prepare_block_strategy(pstrat, stats, blocks)
            continue
        got = P.prepare_block_strategy(pstrat, stats, blocks)
        assert got.label_to_size_map == want["label_to_size_map"]
        assert got.allocation_ordered == want["allocation_ordered"]
        assert got.block_sizes == want["block_sizes"]
        assert got.label_to_block_id == want["label_to_block_id"]
        assert got.transfer_to_compute_map == want["transfer_to_compute_map"]


def test_reverse_map_rejects_two_producers():
    assert P.reverse_transfer_to_compute_map({"a": "b", "c": "d"}) == {"b": "a", "d": "c"}
    with pytest.raises(ValueError, match="mapped from both"):
        P.reverse_transfer_to_compute_map({"a": "b", "c": "b"})


def test_remap_strategy():
    assert P.remap_strategy({"a": [1], "b": [2]}, {"a": "x", "c": "y"}) == {"b": [2], "x": [1]}
    assert P.remap_strategy(None, {"a": "b"}) == {}
    assert P.remap_strategy({"a": [1]}, {"a": "a"}) == {"a": [1]}
