"""Offload-timing aggregation: the oracle pinned by the reference's fixtures, the product against the oracle.

Fixtures transcribed from tests/unit/test_offload_timing_collector.py:538-631
(snapshot totals, report sums and averages, per-trap min/max/avg/median/std).
"""

from __future__ import annotations

import math
import random
import statistics

import pytest

from flextensor_amd.timing import OffloadTimingSnapshot, TrapTimingRecord, build_report, hidden_fraction
from oracle import timing as otim


def _snap(rows):
    return OffloadTimingSnapshot([TrapTimingRecord(label, transfer_ms=t, compute_ms=c, wait_ms=w)
                                  for label, t, c, w in rows])


def test_oracle_snapshot_totals_fixture():
    # test_offload_timing_collector.py:538-547: a (t1, c2, w3) + b (t4, c5, w6)
    assert otim.pass_totals([("a", 1.0, 2.0, 3.0), ("b", 4.0, 5.0, 6.0)]) == (5.0, 7.0, 9.0)


def test_oracle_report_fixture():
    # test_offload_timing_collector.py:578-631
    passes = [[("L0", 10.0, 1.0, 100.0), ("L1", 20.0, 2.0, 200.0)],
              [("L0", 30.0, 3.0, 300.0), ("L1", 40.0, 4.0, 400.0)],
              [("L0", 50.0, 5.0, 500.0), ("L1", 80.0, 8.0, 800.0)]]
    st = otim.per_trap_stats(passes)
    assert list(st) == ["L0", "L1"]
    for label, c in (("L0", [1.0, 3.0, 5.0]), ("L1", [2.0, 4.0, 8.0])):
        mn, mx, avg, med, std = st[label]["compute"]
        assert (mn, mx, avg, med) == (min(c), max(c), sum(c) / 3, statistics.median(c))
        assert math.isclose(std, statistics.stdev(c), rel_tol=1e-12)
    assert st["L1"]["wait"][:4] == (200.0, 800.0, 1400.0 / 3, 400.0)


def test_oracle_hidden_fraction_closed_forms():
    assert otim.hidden_fraction([[("a", 4.0, 9.0, 0.0)]]) == 1.0  # nothing waited: fully hidden
    assert otim.hidden_fraction([[("a", 4.0, 9.0, 1.0)], [("a", 4.0, 9.0, 1.0)]]) == 0.75
    assert otim.hidden_fraction([[("a", 4.0, 0.0, 8.0)]]) == 0.0  # clipped
    assert otim.hidden_fraction([]) == 1.0


def test_product_report_matches_reference_fixture():
    # test_offload_timing_collector.py:548-567: passes a (w1, t2, c3) and a (w3, t4, c5)
    rep = build_report([_snap([("a", 2.0, 3.0, 1.0)]), _snap([("a", 4.0, 5.0, 3.0)])])
    assert rep.num_passes == 2
    assert (rep.total_wait_sum, rep.total_transfer_sum, rep.total_compute_sum) == (4.0, 6.0, 8.0)
    assert (rep.total_wait_avg, rep.total_transfer_avg, rep.total_compute_avg) == (2.0, 3.0, 4.0)


@pytest.mark.parametrize("seed", range(5))
def test_product_report_matches_oracle(seed):
    rng = random.Random(seed)
    labels = [f"layers.{i}" for i in range(rng.randint(1, 6))]
    passes = [[(lb, rng.uniform(0, 20), rng.uniform(0, 50), rng.choice([0.0, rng.uniform(0, 5)])) for lb in labels]
              for _ in range(rng.randint(1, 7))]
    rep = build_report([_snap(p) for p in passes])
    want = otim.per_trap_stats(passes)
    assert [s.label for s in rep.per_trap] == list(want)
    for s in rep.per_trap:
        for col in ("compute", "transfer", "wait"):
            got = tuple(getattr(s, f"{col}_{k}") for k in ("min", "max", "avg", "median", "std"))
            assert all(math.isclose(g, w, rel_tol=1e-9, abs_tol=1e-12) for g, w in zip(got, want[s.label][col]))
    assert math.isclose(rep.hidden_fraction, otim.hidden_fraction(passes), rel_tol=1e-12, abs_tol=1e-15)
    assert math.isclose(hidden_fraction(rep.total_wait_sum, rep.total_transfer_sum), otim.hidden_fraction(passes),
                        rel_tol=1e-12, abs_tol=1e-15)


def test_compute_budget_prefers_median_then_mean_then_min():
    rep = build_report([_snap([("a", 1.0, 4.0, 0.0)]), _snap([("a", 1.0, 6.0, 0.0)]), _snap([("a", 1.0, 2.0, 0.0)])])
    st = rep.per_trap[0]
    assert st.compute_budget_ms() == 4.0 and st.compute_budget_ms(conservative=True) == 2.0
    assert build_report([_snap([("a", 1.0, 0.0, 0.0)])]).per_trap[0].compute_budget_ms() == 0.0
