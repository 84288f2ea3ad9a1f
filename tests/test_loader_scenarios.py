"""Ordering scenarios of the two pipelined loaders on recording fake streams (no GPU).

Restates the reference's scenario suites for PreallocatedBatchTransferTensorLoader
and ...Reordered (tests/unit/test_loader_synchronization.py:442-1560):
  * a compute-stream wait precedes every streamed label's forward (simple
    pipelines, gap labels, leading and mixed gaps), and a slow transfer stalls
    there and not only after the read;
  * a slot is overwritten only after the transfer stream waited for its last use;
  * gap labels schedule nothing and still record their compute event;
  * one fork per forward at the first label, one join at the last, a second
    fork after a piece join, and the join of one pass precedes the next fork;
  * event maps are empty after the last label, and a later request never
    waits on an earlier request's events;
  * the timing hooks pair up, with the wait after compute_end (default) or
    before compute_start (reordered).
"""

from __future__ import annotations

import logging

import pytest

from flextensor_amd.loaders import PreallocatedBatchTransferTensorLoader, PreallocatedBatchTransferTensorLoaderReordered
from flextensor_amd.planner import LayerStatistics, TensorStatistics
from flextensor_amd.timing import OffloadTimingCollector
from tests.fakes import FakeBackend, FakeController, Recorder

KINDS = {"default": PreallocatedBatchTransferTensorLoader, "reordered": PreallocatedBatchTransferTensorLoaderReordered}
BOTH = pytest.mark.parametrize("kind", list(KINDS))

# embed -> L0 -> L1 -> L2 over two slots (L1 reuses embed's slot 0)
SIMPLE = (["embed", "L0", "L1", "L2"], {"embed": "L0", "L0": "L1", "L1": "L2"}, {"embed": 0, "L0": 1, "L1": 0})
SHORT = (["embed", "L0", "L1"], {"embed": "L0", "L0": "L1"}, {"embed": 0, "L0": 1})
GAP_CASES = {
    # labels, gap labels, transfer -> compute, slots, the label after the gaps
    "single": (["embed", "L0", "L1", "L2", "L3"], {"L2"}, {"embed": "L0", "L0": "L1", "L1": "L3"},
               {"embed": 0, "L0": 1, "L1": 0}, "L3"),
    "consecutive": (["embed", "L0", "L1", "L2", "L3", "L4"], {"L2", "L3"}, {"embed": "L0", "L0": "L1", "L1": "L4"},
                    {"embed": 0, "L0": 1, "L1": 0}, "L4"),
    "leading": (["embed", "L0", "L1", "L2", "L3"], {"L0", "L1", "L2"}, {"embed": "L3"}, {"embed": 0}, "L3"),
}
LONG = ["embed"] + [f"L{i}" for i in range(9)]


def _loader(kind, labels, t2c, l2b, *, gaps=(), slow=False, collector=None):
    rec = Recorder()
    backend = FakeBackend(rec, slow_transfer=slow)
    ctrl = FakeController(rec, backend)
    t = TensorStatistics(tensor_id=1, name="t", size_bytes=1024, load_time_ms=0.1)
    stats = [LayerStatistics(x, [] if x in gaps else [t], 1.0) for x in labels]
    loader = KINDS[kind](stats, None, l2b, t2c, ctrl, collector, None, backend=backend)
    rec.log.clear()
    rec.counter = 0
    return loader, rec


def _run(loader, rec, labels):
    for x in labels:
        loader.enter(x)
        rec.forward(x)
        loader.exit(x)


def _forward(rec, label, nth=0):
    return rec.find("forward", target=label)[nth]


def _compute_waits(rec, *, before=None, after=-1, stalled=None):
    return [i for i, e in enumerate(rec.log)
            if e.op == "wait_event" and e.stream == "compute" and after < i < (before if before is not None else 10**9)
            and (stalled is None or e.stalled == stalled)]


def _pairs(rec, first, second):
    """Indices i where log[i] is (op, stream) ``first`` and log[i + 1] is ``second``."""
    return [i for i, (a, b) in enumerate(zip(rec.log, rec.log[1:]))
            if (a.op, a.stream) == first and (b.op, b.stream) == second]


FORK = (("record_event", "compute"), ("wait_event", "transfer"))
JOIN = (("record_event", "transfer"), ("wait_event", "compute"))


def _mixed_gap_maps(gaps):
    off = [x for x in LONG if x not in gaps]
    t2c = {off[i]: off[i + 1] for i in range(len(off) - 1)}
    return off, t2c, {t: i % 2 for i, t in enumerate(t2c)}


# ---- waits before reads ----------------------------------------------------------------


@BOTH
@pytest.mark.parametrize("slow", [False, True])
def test_simple_pipeline_waits_before_every_read(kind, slow):
    labels, t2c, l2b = SIMPLE
    loader, rec = _loader(kind, labels, t2c, l2b, slow=slow)
    _run(loader, rec, labels)
    for x in labels[1:]:
        fwd = _forward(rec, x)
        assert _compute_waits(rec, before=fwd, stalled=True if slow else None), rec.dump()
    if not slow:  # transfers that finish in time never stall a wait
        assert not [e for e in rec.log if e.op == "wait_event" and e.stalled], rec.dump()


@pytest.mark.parametrize("kind", ["reordered"])
def test_reordered_wait_is_in_enter_of_the_reader(kind):
    """The reordered loader's wait for a label's data sits between the previous forward and this one
    (in enter), not only after the read."""
    labels, t2c, l2b = SIMPLE
    loader, rec = _loader(kind, labels, t2c, l2b, slow=True)
    _run(loader, rec, labels)
    for prev, x in zip(labels, labels[1:]):
        assert _compute_waits(rec, before=_forward(rec, x), after=_forward(rec, prev), stalled=True), rec.dump()


@BOTH
@pytest.mark.parametrize("case", list(GAP_CASES))
def test_gaps_schedule_nothing_and_the_next_read_waits(kind, case):
    labels, gaps, t2c, l2b, target = GAP_CASES[case]
    loader, rec = _loader(kind, labels, t2c, l2b, gaps=gaps, slow=True)
    _run(loader, rec, labels)
    for g in gaps:
        assert not rec.find("schedule_transfer", target=g), rec.dump()
    assert _compute_waits(rec, before=_forward(rec, target), stalled=True), rec.dump()
    # while a gap label runs (its enter to its exit), no transfer is scheduled
    for g in sorted(gaps):
        fwd = _forward(rec, g)
        nxt = min(i for i in rec.find("forward") if i > fwd) if any(i > fwd for i in rec.find("forward")) else len(rec.log)
        assert not [i for i in rec.find("schedule_transfer") if fwd < i < nxt and rec.log[i].target in gaps]


def test_reordered_gap_label_adds_no_data_wait():
    """A gap label consumes no transfer, so the reordered loader's enter for it waits on nothing."""
    labels, gaps, t2c, l2b, _ = GAP_CASES["single"]
    loader, rec = _loader("reordered", labels, t2c, l2b, gaps=gaps)
    loader_labels = labels[: labels.index("L2")]
    _run(loader, rec, loader_labels)
    mark = len(rec.log)
    loader.enter("L2")
    assert _compute_waits(rec, after=mark - 1) == [], rec.dump()


def test_default_gap_label_records_its_compute_event():
    """The default loader records a compute event for a gap label too (slot reuse is ordered on it)."""
    labels, gaps, t2c, l2b, _ = GAP_CASES["single"]
    loader, rec = _loader("default", labels, t2c, l2b, gaps=gaps)
    _run(loader, rec, labels)
    between = [i for i in rec.find("record_event", stream="compute") if _forward(rec, "L2") < i < _forward(rec, "L3")]
    assert between, rec.dump()


@BOTH
@pytest.mark.parametrize("gaps", [{"L2", "L5", "L6"}, {"L2", "L3"}, {"L3", "L4", "L5"}],
                         ids=["single+double", "consecutive-double", "consecutive-triple"])
def test_mixed_gaps_in_a_ten_label_model(kind, gaps):
    off, t2c, l2b = _mixed_gap_maps(gaps)
    loader, rec = _loader(kind, LONG, t2c, l2b, gaps=gaps, slow=True)
    _run(loader, rec, LONG)
    for x in off[1:]:
        assert _compute_waits(rec, before=_forward(rec, x), stalled=True), (x, rec.dump())
    for g in gaps:
        assert not rec.find("schedule_transfer", target=g)
    if kind == "default":
        assert len(rec.find("record_event", stream="compute")) >= len(LONG)


# ---- slot reuse --------------------------------------------------------------------------


@BOTH
def test_slot_reuse_waits_for_its_last_use(kind):
    """L1 reuses embed's slot: the transfer stream waits before schedule_transfer(L1), after L0 read the slot."""
    labels, t2c, l2b = SIMPLE
    loader, rec = _loader(kind, labels, t2c, l2b)
    _run(loader, rec, labels)
    sched_l1 = rec.find("schedule_transfer", target="L1")[0]
    waits = [i for i in rec.find("wait_event", stream="transfer") if i < sched_l1]
    assert waits, rec.dump()
    # the awaited event was recorded on the compute stream after L0's forward (the slot's last reader)
    awaited = rec.log[waits[-1]].target
    recorded = [i for i, e in enumerate(rec.log) if e.op == "record_event" and e.target == awaited]
    assert recorded and rec.log[recorded[0]].stream == "compute" and recorded[0] > _forward(rec, "L0"), rec.dump()


# ---- fork / join ------------------------------------------------------------------------


@BOTH
def test_one_fork_at_the_first_label_and_one_join_at_the_last(kind):
    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b)
    _run(loader, rec, labels)
    assert [(e.op, e.stream) for e in rec.log[:2]] == list(FORK), rec.dump()
    assert [(e.op, e.stream) for e in rec.log[-2:]] == list(JOIN), rec.dump()
    assert len(_pairs(rec, *FORK)) == 1


@BOTH
def test_join_of_one_pass_precedes_the_next_fork(kind):
    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b)
    _run(loader, rec, labels)
    _run(loader, rec, labels)
    last1, first2 = rec.find("forward")[len(labels) - 1], rec.find("forward")[len(labels)]
    joins = [i for i in _pairs(rec, *JOIN) if i > last1]
    forks = [i for i in _pairs(rec, *FORK) if last1 < i < first2]
    assert joins and forks and joins[0] < forks[0], rec.dump()


@BOTH
def test_post_only_last_label_exit_skips_the_cross_piece_join(kind):
    """A piece that holds only the last label's exit: no transfer join, no compute wait, nothing outstanding."""
    labels, t2c, l2b = ["embed", "L0"], {"embed": "L0"}, {"embed": 0}
    loader, rec = _loader(kind, labels, t2c, l2b)
    loader.enter("L0")
    loader.join_after_forward()
    rec.log.clear()
    policy = loader.piecewise_prefetch_policy
    policy.enabled, policy.strict = True, True
    policy.on_wait("L0")
    policy.on_schedule("L0", "L0")
    loader.exit("L0")
    assert len(rec.find("record_event", stream="compute")) == 1, rec.dump()
    assert rec.find("record_event", stream="transfer") == [] and rec.find("wait_event", stream="compute") == []
    assert policy.on_piece_join() == []
    assert loader.scheduled_transfers == {}


# ---- event maps and repeated requests --------------------------------------------------


@BOTH
def test_first_enter_is_silent_when_the_maps_are_empty(kind, caplog):
    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b)
    assert not loader._transfer_runtime.is_active
    with caplog.at_level(logging.DEBUG, logger="flextensor_amd.loaders"):
        loader.enter("embed")
    assert all("stale" not in r.getMessage().lower() and "abort" not in r.getMessage().lower()
               for r in caplog.records)


@BOTH
@pytest.mark.parametrize("slow", [False, True])
def test_second_request_never_waits_on_the_first_requests_events(kind, slow):
    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b, slow=slow)
    _run(loader, rec, labels)
    assert loader.scheduled_transfers == {} and loader._transfer_runtime._last_use_by_slot == {}
    first = {e.target for e in rec.log if e.op == "record_event" and e.stream == "transfer"}
    split = len(rec.log)
    _run(loader, rec, labels)
    assert loader.scheduled_transfers == {}
    assert [e for e in rec.log[split:] if e.op == "wait_event" and e.stream == "compute" and e.target in first] == []
    if slow:
        assert _compute_waits(rec, before=split, stalled=True), rec.dump()


def test_reordered_preload_counts_as_consumed_by_a_strict_policy():
    """Two passes of a cyclic reordered schedule under a strict piecewise policy raise nothing."""
    labels = ["embed", "L0", "L1"]
    loader, rec = _loader("reordered", labels, {"embed": "L0", "L0": "L1", "L1": "embed"},
                          {"embed": 0, "L0": 1, "L1": 2})
    loader.piecewise_prefetch_policy.enabled = True
    loader.piecewise_prefetch_policy.strict = True
    _run(loader, rec, labels)
    _run(loader, rec, labels)
    assert loader.scheduled_transfers == {}


# ---- timing hooks ------------------------------------------------------------------------


def _hook_calls(kind):
    calls = []
    spy = OffloadTimingCollector(enabled=False)
    for name in ("on_pass_start", "record_transfer_start", "record_transfer_end", "record_compute_start",
                 "record_compute_end", "record_wait_start", "record_wait_end"):
        setattr(spy, name, (lambda n: lambda *a, **k: calls.append((n, a)))(name))
    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b, collector=spy)
    _run(loader, rec, labels)
    return calls, loader.transfer_stream, set(l2b), labels


@BOTH
def test_timing_hooks_carry_labels_and_the_transfer_stream(kind):
    calls, stream, streamed, labels = _hook_calls(kind)
    names = [n for n, _ in calls]
    assert names[0] == "on_pass_start" and names.count("on_pass_start") == 1
    for n, a in calls:
        if n in ("record_transfer_start", "record_transfer_end"):
            assert a[0] in streamed and a[1] is stream
    assert {a[0] for n, a in calls if n == "record_compute_start"} == set(labels)
    assert {a[0] for n, a in calls if n == "record_compute_end"} == set(labels)
    waits = [a[0] for n, a in calls if n == "record_wait_start"]
    assert waits and waits == [a[0] for n, a in calls if n == "record_wait_end"]


def test_default_wait_follows_compute_end():
    calls, *_ = _hook_calls("default")
    for label in [a[0] for n, a in calls if n == "record_wait_start"]:
        end = next(i for i, (n, a) in enumerate(calls) if n == "record_compute_end" and a[0] == label)
        assert any(n == "record_wait_start" and a[0] == label for n, a in calls[end + 1:]), calls


def test_reordered_wait_precedes_compute_start():
    calls, *_ = _hook_calls("reordered")
    for label in [a[0] for n, a in calls if n == "record_wait_start"]:
        w = next(i for i, (n, a) in enumerate(calls) if n == "record_wait_start" and a[0] == label)
        c = next(i for i, (n, a) in enumerate(calls) if n == "record_compute_start" and a[0] == label)
        assert w < c, calls


@BOTH
def test_shutdown_synchronizes_before_the_blocks_go(kind):
    """test_loaders_pin_fallback.py:287-299: the transfer stream is synchronized before the controller
    releases the blocks its copies read."""
    from tests.fakes import Entry

    labels, t2c, l2b = SHORT
    loader, rec = _loader(kind, labels, t2c, l2b)
    loader.allocation_controller.shutdown = lambda: rec.log.append(Entry("shutdown", "host", "controller"))
    _run(loader, rec, labels)
    rec.log.clear()
    loader.shutdown()
    assert [(e.op, e.stream) for e in rec.log][-2:] == [("synchronize", "transfer"), ("shutdown", "host")], rec.dump()
