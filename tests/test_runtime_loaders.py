"""Transfer runtime and pipelined loaders on recording fake streams (no GPU).

The runtime tests restate the reference's runtime contract
(tests/unit/core/test_transfer.py); the loader tests pin the frozen trace
(tests/unit/test_loader_synchronization.py:288-363) and compare full
operation traces with the oracle across gap patterns, cyclic preloads,
several passes and abort recovery.
"""

from __future__ import annotations

import json
import logging
import random
from pathlib import Path

import pytest

from flextensor_amd.loaders import PreallocatedBatchTransferTensorLoader, PreallocatedBatchTransferTensorLoaderReordered
from flextensor_amd.planner import LayerStatistics, TensorStatistics
from flextensor_amd.timing import OffloadTimingCollector
from flextensor_amd.transfer import HipTransferRuntime, TransferStreamSynchronizationError
from oracle import schedule as osch
from tests.fakes import FakeBackend, FakeController, Recorder

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_cases.json").read_text())
LOADERS = {"default": PreallocatedBatchTransferTensorLoader, "reordered": PreallocatedBatchTransferTensorLoaderReordered}


@pytest.fixture
def rt():
    rec = Recorder()
    backend = FakeBackend(rec)
    return HipTransferRuntime(None, backend=backend), rec, backend


# ---- runtime ---------------------------------------------------------------


def test_same_slot_reuse_waits_for_last_use(rt):
    runtime, rec, backend = rt
    runtime.begin()
    first = runtime.submit("slot-0", lambda: rec.log.append(_e("copy", "first")))
    runtime.wait_ready(first)
    runtime.finish_use("slot-0")
    last_use = next(e.target for e in reversed(rec.log) if (e.op, e.stream) == ("record_event", "compute"))
    runtime.submit("slot-0", lambda: rec.log.append(_e("copy", "second")))
    wait = next(i for i, e in enumerate(rec.log) if (e.op, e.stream, e.target) == ("wait_event", "transfer", last_use))
    copy = next(i for i, e in enumerate(rec.log) if e.target == "second")
    assert wait < copy


def _e(op, target):
    from tests.fakes import Entry

    return Entry(op, "transfer", target)


def test_no_cross_slot_wait(rt):
    runtime, rec, _ = rt
    runtime.begin()
    runtime.submit("slot-0", lambda: None)
    runtime.submit("slot-1", lambda: None)
    assert len(rec.find("wait_event", stream="transfer")) == 1  # only the fork


def test_transfer_runs_on_transfer_stream(rt):
    runtime, rec, backend = rt
    seen = []
    runtime.begin()
    runtime.submit(0, lambda: seen.append(backend.current_stream().name))
    assert seen == ["transfer"] and backend.current_stream().name == "compute"


def test_ticket_repr(rt):
    runtime, _, _ = rt
    runtime.begin()
    t = runtime.submit("slot", lambda: None, trace_label="schedule=embed consume=L0")
    assert repr(t) == "TransferTicket(slot='slot', trace_label='schedule=embed consume=L0')"


def test_busy_slot_rejected(rt):
    runtime, _, _ = rt
    runtime.begin()
    active = runtime.submit("slot", lambda: None, trace_label="x")
    with pytest.raises(RuntimeError, match="still in use") as caught:
        runtime.submit("slot", lambda: None)
    assert repr(active) in str(caught.value)


def test_foreign_and_stale_tickets(rt):
    runtime, rec, backend = rt
    other = HipTransferRuntime(None, backend=backend)
    runtime.begin()
    other.begin()
    t = runtime.submit("slot", lambda: None)
    with pytest.raises(ValueError, match="different"):
        other.wait_ready(t)
    runtime.wait_ready(t)
    runtime.finish_use("slot")
    cur = runtime.submit("slot", lambda: None)
    runtime.wait_ready(cur)
    with pytest.raises(ValueError, match="stale") as caught:
        runtime.wait_ready(t)
    assert repr(t) in str(caught.value)
    runtime.join()
    with pytest.raises(ValueError, match="stale"):
        runtime.wait_ready(cur)


def test_host_wait_blocks_the_host_and_leaves_the_stream_unordered(rt):
    runtime, rec, backend = rt
    runtime.begin()
    ticket = runtime.submit("slot-0", lambda: None)
    rec.log.clear()
    runtime.wait_ready(ticket, host=True)
    assert rec.triples() == [("synchronize_event", "host", ticket._event.name)]
    backend.capturing = True  # a captured transfer has not run: the stream waits
    rec.log.clear()
    runtime.wait_ready(ticket, host=True)
    assert rec.triples() == [("wait_event", "compute", ticket._event.name)]
    backend.capturing = False
    runtime.finish_use("slot-0")
    runtime.submit("slot-0", lambda: None)
    with pytest.raises(ValueError, match="stale"):  # the ticket checks hold for host waits too
        runtime.wait_ready(ticket, host=True)
    foreign = HipTransferRuntime(None, backend=backend)
    foreign.begin()
    with pytest.raises(ValueError, match="different"):
        runtime.wait_ready(foreign.submit("slot-0", lambda: None), host=True)


def test_lifecycle_errors(rt):
    runtime, rec, _ = rt
    with pytest.raises(RuntimeError, match="begin"):
        runtime.submit(0, lambda: None)
    with pytest.raises(RuntimeError, match="begin"):
        runtime.finish_use(0)
    assert not runtime.is_active
    runtime.begin()
    assert runtime.is_active
    with pytest.raises(RuntimeError, match="already active"):
        runtime.begin()
    runtime.join()
    assert not runtime.is_active
    runtime.close()
    runtime.close()
    assert [(e.op, e.stream) for e in rec.log].count(("synchronize", "transfer")) == 1
    with pytest.raises(RuntimeError, match="closed"):
        runtime.begin()


def test_callback_error_propagates(rt):
    runtime, _, _ = rt
    runtime.begin()

    def fail():
        raise LookupError("copy failed")

    with pytest.raises(LookupError, match="copy failed"):
        runtime.submit("slot", fail)


@pytest.mark.parametrize("which", ["record_event", "wait_event"])
def test_join_wraps_stream_errors(rt, which):
    runtime, _, backend = rt
    runtime.begin()
    (backend.transfer if which == "record_event" else backend.compute).fail_on.add(which)
    with pytest.raises(TransferStreamSynchronizationError, match=which) as caught:
        runtime.join()
    assert isinstance(caught.value.__cause__, RuntimeError)


def test_close_wraps_sync_error(rt):
    runtime, _, backend = rt
    backend.transfer.fail_on.add("synchronize")
    with pytest.raises(TransferStreamSynchronizationError, match="synchronize failed"):
        runtime.close()


# ---- loaders -----------------------------------------------------------------


def _stats(labels, gaps=()):
    t = TensorStatistics(tensor_id=1, name="t", size_bytes=1024, load_time_ms=0.1)
    return [LayerStatistics(x, [] if x in gaps else [t], 1.0) for x in labels]


def _make(kind, labels, t2c, l2b, slow=False, gaps=(), collector=None):
    rec = Recorder()
    backend = FakeBackend(rec, slow_transfer=slow)
    ctrl = FakeController(rec, backend)
    loader = LOADERS[kind](_stats(labels, gaps), None, l2b, t2c, ctrl, collector, None, backend=backend)
    rec.log.clear()
    rec.counter = 0
    return loader, rec, ctrl


def _run(loader, rec, labels, passes=1):
    for _ in range(passes):
        for x in labels:
            loader.enter(x)
            rec.forward(x)
            loader.exit(x)


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_frozen_trace(kind):
    c = GOLD["frozen_trace"]
    loader, rec, ctrl = _make(kind, c["labels"], c["transfer_to_compute_map"], c["label_to_block_id"])
    _run(loader, rec, c["labels"])
    assert [list(x) for x in rec.ops()] == c["expected"][kind]
    assert set(ctrl.streams_seen) == {"transfer"}


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_ticket_trace_label(kind):
    c = GOLD["ticket_trace_label"]
    loader, rec, _ = _make(kind, c["labels"], c["transfer_to_compute_map"], c["label_to_block_id"])
    loader.enter("embed")
    scheduled = next(iter(loader.scheduled_transfers.values()))
    ticket = scheduled[0] if isinstance(scheduled, list) else scheduled
    assert ticket.trace_label == c["expected"]


def _pipeline(labels, gaps, blocks, cyclic):
    off = [x for x in labels if x not in gaps]
    t2c = {off[i]: off[i + 1] for i in range(len(off) - 1)}
    if cyclic and len(off) > 2:
        t2c[off[-1]] = off[0]
    l2b = {t: i % blocks for i, t in enumerate(t2c)}
    return t2c, l2b


@pytest.mark.parametrize("kind", ["default", "reordered"])
@pytest.mark.parametrize("seed", range(30))
def test_traces_match_oracle(kind, seed):
    rng = random.Random(seed)
    n = rng.randrange(2, 11)
    labels = ["embed"] + [f"L{i}" for i in range(n - 1)]
    gaps = set(rng.sample(labels[1:], rng.randrange(0, max(1, n // 3))))
    blocks = rng.choice([2, 3])
    cyclic = kind == "reordered" and rng.random() < 0.5
    t2c, l2b = _pipeline(labels, gaps, blocks, cyclic)
    passes = rng.choice([1, 2, 3])
    loader, rec, _ = _make(kind, labels, t2c, l2b, gaps=gaps)
    _run(loader, rec, labels, passes)
    want = osch.trace(kind, labels, t2c, l2b, osch.passes(labels, passes))
    assert rec.triples() == want


def _ready_waits(rec, op, stream):
    """(ordinal of the transfer, forwards run before the wait) for each wait ``op`` on ``stream`` on a ready event."""
    ready, pending, count, forwards, waits = {}, None, 0, 0, []
    for e in rec.log:
        if e.op == "schedule_transfer":
            pending, count = count, count + 1
        elif (e.op, e.stream) == ("record_event", "transfer") and pending is not None:
            ready[e.target], pending = pending, None  # the submit records its ready event right after the copy
        elif e.op == "forward":
            forwards += 1
        elif (e.op, e.stream) == (op, stream) and e.target in ready:
            waits.append((ready[e.target], forwards))
    return waits


@pytest.mark.parametrize("seed", range(30))
def test_host_waited_reordered_loader_waits_the_same_copies_on_the_host(seed):
    """With ``link_bound`` the reordered loader issues the same copies in the same order, waits for each
    consumed copy on the host before the same forward as the stream-waited loader does on the compute
    stream, never makes the compute stream wait on a copy, and queues each label's copy before it blocks."""
    rng = random.Random(seed)
    n = rng.randrange(2, 11)
    labels = ["embed"] + [f"L{i}" for i in range(n - 1)]
    gaps = set(rng.sample(labels[1:], rng.randrange(0, max(1, n // 3))))
    t2c, l2b = _pipeline(labels, gaps, rng.choice([2, 3]), rng.random() < 0.5)
    passes = rng.choice([1, 2, 3])
    streamed, s_rec, _ = _make("reordered", labels, t2c, l2b, slow=True, gaps=gaps)
    _run(streamed, s_rec, labels, passes)
    hosted, h_rec, _ = _make("reordered", labels, t2c, l2b, slow=True, gaps=gaps)
    hosted.link_bound = True
    _run(hosted, h_rec, labels, passes)
    copies = [e.target for e in h_rec.log if e.op == "schedule_transfer"]
    assert copies == [e.target for e in s_rec.log if e.op == "schedule_transfer"]
    waited = _ready_waits(s_rec, "wait_event", "compute")
    assert _ready_waits(h_rec, "synchronize_event", "host") == waited
    assert _ready_waits(h_rec, "wait_event", "compute") == []
    assert _host_waited_before_use(h_rec, t2c), h_rec.dump()
    # between two forwards, the copy scheduled there is queued before the host blocks
    segment: list = []
    for e in [*h_rec.log, None]:
        if e is None or e.op == "forward":
            ops = [x.op for x in segment]
            if "schedule_transfer" in ops and "synchronize_event" in ops:
                assert ops.index("schedule_transfer") < ops.index("synchronize_event"), h_rec.dump()
            segment = []
        else:
            segment.append(e)
    assert not hosted.scheduled_transfers and not hosted._transfer_runtime.is_active


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_link_bound_keeps_the_reference_trace_under_capture(kind):
    """Under graph capture a link-bound loader keeps the reference's order and stream waits."""
    labels = ["embed"] + [f"L{i}" for i in range(6)]
    t2c, l2b = _pipeline(labels, {"L2"}, 2, kind == "reordered")
    loader, rec, _ = _make(kind, labels, t2c, l2b, gaps={"L2"})
    loader.link_bound = True
    loader.backend.capturing = True
    _run(loader, rec, labels, 2)
    assert rec.triples() == osch.trace(kind, labels, t2c, l2b, osch.passes(labels, 2))
    assert not rec.find("synchronize_event")


@pytest.mark.parametrize("seed", range(30))
def test_link_bound_default_loader_releases_before_its_wait(seed):
    """A link-bound default loader issues the same copies in the same order and makes the compute stream
    wait for each before the same forward as the reference's order, but records the release of the slots
    a label read before that wait, so the copy into one of them can queue behind the awaited one."""
    rng = random.Random(seed)
    n = rng.randrange(2, 11)
    labels = ["embed"] + [f"L{i}" for i in range(n - 1)]
    gaps = set(rng.sample(labels[1:], rng.randrange(0, max(1, n // 3))))
    t2c, l2b = _pipeline(labels, gaps, rng.choice([2, 3]), False)
    passes = rng.choice([1, 2, 3])
    ref, r_rec, _ = _make("default", labels, t2c, l2b, slow=True, gaps=gaps)
    _run(ref, r_rec, labels, passes)
    early, e_rec, _ = _make("default", labels, t2c, l2b, slow=True, gaps=gaps)
    early.link_bound = True
    _run(early, e_rec, labels, passes)
    assert [e.target for e in e_rec.log if e.op == "schedule_transfer"] == \
        [e.target for e in r_rec.log if e.op == "schedule_transfer"]
    assert _ready_waits(e_rec, "wait_event", "compute") == _ready_waits(r_rec, "wait_event", "compute")
    assert sorted(e_rec.ops()) == sorted(r_rec.ops())  # the same operations, reordered
    # within each exit (between a forward and the next schedule or forward), the compute stream's release
    # record precedes its wait on a transfer; in the reference's order it follows it
    for rec, release_first in ((e_rec, True), (r_rec, False)):
        ready, pending = set(), False
        for e in rec.log:  # a submit records its ready event right after the copy
            if e.op == "schedule_transfer":
                pending = True
            elif (e.op, e.stream) == ("record_event", "transfer") and pending:
                ready.add(e.target)
                pending = False
        segment: list = []
        for e in [*rec.log, None]:
            if e is None or e.op in ("forward", "schedule_transfer"):
                ops = [(x.op, x.stream, x.target in ready) for x in segment]
                waits = [i for i, (op, st, is_ready) in enumerate(ops) if (op, st, is_ready) == ("wait_event", "compute", True)]
                releases = [i for i, (op, st, _) in enumerate(ops) if (op, st) == ("record_event", "compute")]
                if waits and releases:
                    assert (releases[0] < waits[0]) == release_first, rec.dump()
                segment = []
            else:
                segment.append(e)
    assert not early.scheduled_transfers and not early._transfer_runtime.is_active


def _host_waited_before_use(rec, t2c) -> bool:
    """Every copy a unit consumes is host-synchronized before the unit's forward, unless a join (the
    compute stream waiting on the transfer stream's tail) ordered it first."""
    pending: dict = {}  # consumer -> ready events not yet ordered before it
    waited, last_schedule, ready = set(), None, set()
    for e in rec.log:
        if e.op == "schedule_transfer":
            last_schedule = e.target
        elif (e.op, e.stream) == ("record_event", "transfer") and last_schedule is not None:
            pending.setdefault(t2c[last_schedule], []).append(e.target)
            ready.add(e.target)
            last_schedule = None
        elif e.op == "synchronize_event":
            waited.add(e.target)
        elif (e.op, e.stream) == ("wait_event", "compute") and e.target not in ready:
            pending.clear()  # a join: everything queued before it is ordered
        elif e.op == "forward":
            if any(ev not in waited for ev in pending.pop(e.target, [])):
                return False
    return True


def test_link_bound_abort_recovery_reloads_and_waits_on_the_host():
    """A link-bound reordered pass that stops early leaves copies in flight; the next pass joins, loads
    its first slots again, and blocks the host on every copy a unit consumes before that unit runs."""
    labels = ["L0", "L1", "L2", "L3"]
    t2c = {"L0": "L1", "L1": "L2", "L2": "L3", "L3": "L0"}
    l2b = {"L0": 0, "L1": 1, "L2": 0, "L3": 1}
    loader, rec, _ = _make("reordered", labels, t2c, l2b, slow=True)
    loader.link_bound = True
    for op, x in [("enter", "L0"), ("forward", "L0"), ("exit", "L0"), ("enter", "L1")]:  # stops in L1
        getattr(loader, op)(x) if op != "forward" else rec.forward(x)
    rec.log.clear()
    _run(loader, rec, labels, 2)
    assert [e.target for e in rec.log if e.op == "schedule_transfer"][0] == "L3"  # L0's slot loaded again
    assert _ready_waits(rec, "wait_event", "compute") == []
    assert _host_waited_before_use(rec, t2c), rec.dump()
    assert rec.find("synchronize_event")


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_abort_recovery_joins_then_clears(kind, caplog):
    labels = ["embed", "L0", "L1"]
    t2c, l2b = {"embed": "L0", "L0": "L1"}, {"embed": 0, "L0": 1}
    loader, rec, _ = _make(kind, labels, t2c, l2b)
    loader.enter("embed")
    stale = next(iter(loader.scheduled_transfers.values()))
    rec.log.clear()
    with caplog.at_level(logging.DEBUG, logger="flextensor_amd.loaders"):
        loader.enter("embed")  # previous pass never exited
    assert stale not in loader.scheduled_transfers.values()
    assert any("abort recovery" in r.getMessage() for r in caplog.records)
    assert rec.find("record_event", stream="transfer") and rec.find("wait_event", stream="compute")
    calls = [("enter", "embed"), ("enter", "embed")]
    assert osch.trace(kind, labels, t2c, l2b, calls, reload_after_abort=True)[-len(rec.log):] == rec.triples()


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_abort_recovery_reloads_the_first_slots(kind):
    """A pass that stopped early never issued the cyclic transfers for the next pass's first labels;
    recovery issues them again before the first label reads its slot."""
    labels = ["L0", "L1", "L2", "L3"]
    t2c = {"L0": "L1", "L1": "L2", "L2": "L3", "L3": "L0"}
    l2b = {"L0": 0, "L1": 1, "L2": 0, "L3": 1}
    loader, rec, ctrl = _make(kind, labels, t2c, l2b)
    calls = [("enter", "L0"), ("forward", "L0"), ("exit", "L0"), ("enter", "L1")]  # the pass stops in L1
    for op, x in calls:
        getattr(loader, op)(x) if op != "forward" else rec.forward(x)
    rec.log.clear()
    loader.enter("L0")  # next pass
    reload = [e for e in rec.log if e.op == "schedule_transfer" and e.target == "L3"]
    assert reload, rec.dump()  # L3 carries L0's weights: issued again
    full = calls + [("enter", "L0")]
    product = osch.trace(kind, labels, t2c, l2b, full, reload_after_abort=True)
    assert product[-len(rec.log):] == rec.triples()
    reference = osch.trace(kind, labels, t2c, l2b, full)
    assert len(reference) < len(product)  # the reference's recovery issues no transfer


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_slow_transfer_stalls_before_read(kind):
    labels = ["embed", "L0", "L1", "L2"]
    c = GOLD["frozen_trace"]
    loader, rec, _ = _make(kind, labels, c["transfer_to_compute_map"], c["label_to_block_id"], slow=True)
    _run(loader, rec, labels)
    for x in ("L0", "L1", "L2"):
        fwd = rec.find("forward", target=x)[0]
        assert any(e.op == "wait_event" and e.stream == "compute" and e.stalled for e in rec.log[:fwd]), rec.dump()


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_maps_cleared_after_last_layer(kind):
    labels = ["embed", "L0", "L1"]
    loader, rec, _ = _make(kind, labels, {"embed": "L0", "L0": "L1"}, {"embed": 0, "L0": 1})
    _run(loader, rec, labels)
    assert loader._transfer_runtime._last_use_by_slot == {} and loader.scheduled_transfers == {}
    assert not loader._transfer_runtime.is_active


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_piece_join_allows_second_fork(kind):
    labels = ["embed", "L0", "L1"]
    loader, rec, _ = _make(kind, labels, {"embed": "L0", "L0": "L1"}, {"embed": 0, "L0": 1})
    loader.enter("embed")
    loader.exit("embed")
    loader.join_after_forward()

    def forks():
        return sum(1 for a, b in zip(rec.log, rec.log[1:])
                   if (a.op, a.stream, b.op, b.stream) == ("record_event", "compute", "wait_event", "transfer"))

    assert forks() == 1
    loader.enter("L0")
    assert forks() == 2


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_sync_prev_onload(kind):
    labels = ["embed", "L0"]
    loader, rec, _ = _make(kind, labels, {"embed": "L0"}, {"embed": 0})
    loader.sync_prev_onload()
    assert [(e.op, e.stream) for e in rec.log] == [("wait_stream", "compute")]


def test_reordered_preload_adds_no_compute_wait():
    labels = ["embed", "L0", "L1"]
    loader, rec, _ = _make("reordered", labels, {"embed": "L0", "L0": "L1", "L1": "embed"},
                           {"embed": 0, "L0": 1, "L1": 2})
    loader.sync_prev_onload()
    rec.log.clear()
    loader.enter("embed")
    assert rec.find("wait_event", stream="compute") == []


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_one_compute_label_releases_every_consumed_slot(kind):
    labels = ["A", "B", "C", "tail"]
    loader, rec, _ = _make(kind, labels, {"A": "C", "B": "C"}, {"A": 0, "B": 1})
    for x in ("A", "B", "C"):
        loader.enter(x)
        loader.exit(x)
    loader._transfer_runtime.submit(0, lambda: None)
    loader._transfer_runtime.submit(1, lambda: None)


@pytest.mark.parametrize("kind", ["default", "reordered"])
def test_timing_hooks_pair_up(kind):
    calls = []

    class Spy(OffloadTimingCollector):
        def __init__(self):
            super().__init__(enabled=False)

    spy = Spy()
    for name in ("on_pass_start", "record_transfer_start", "record_transfer_end", "record_compute_start",
                 "record_compute_end", "record_wait_start", "record_wait_end"):
        setattr(spy, name, (lambda n: lambda *a, **k: calls.append(n))(name))
    labels = ["embed", "L0", "L1"]
    loader, rec, _ = _make(kind, labels, {"embed": "L0", "L0": "L1"}, {"embed": 0, "L0": 1}, collector=spy)
    _run(loader, rec, labels)
    assert calls[0] == "on_pass_start"
    for col in ("transfer", "compute", "wait"):
        starts = [i for i, c in enumerate(calls) if c == f"record_{col}_start"]
        ends = [i for i, c in enumerate(calls) if c == f"record_{col}_end"]
        assert len(starts) == len(ends) > 0 and all(s < e for s, e in zip(starts, ends))


class _ClockEvent:
    """Fake timing event: ``record`` stamps the fake clock; a replay re-stamps through ``clock``."""

    def __init__(self, clock):
        self.clock, self.t = clock, None

    def record(self, stream=None):
        self.t = self.clock["now"]
        self.clock["now"] += self.clock["step"]
        self.clock["recorded"].append(self)
        return self

    def elapsed_time(self, end):
        return end.t - self.t


def _graph_collector(capturing):
    clock = {"now": 0.0, "step": 1.0, "recorded": []}
    col = OffloadTimingCollector(["L0", "L1"], event_factory=lambda: _ClockEvent(clock), current_stream=lambda: None,
                                 synchronize=lambda: None, graph_replay=True, is_capturing=lambda: capturing["on"])
    return col, clock


def _timed_pass(col):
    col.on_pass_start()
    for label in ("L0", "L1"):
        col.record_transfer_start(label, None)
        col.record_transfer_end(label, None)
        col.record_compute_start(label)
        col.record_compute_end(label)
        col.record_wait_start(label)
        col.record_wait_end(label)


def test_graph_replay_timing_reads_each_replay():
    """offload_timing.py:319-352: a captured pass is timed by every replay, read after it."""
    capturing = {"on": False}
    col, clock = _graph_collector(capturing)
    _timed_pass(col)  # eager pass
    capturing["on"] = True
    _timed_pass(col)  # the captured pass: recorded once, read never
    assert col.flush() is False and col.snapshots == []
    capturing["on"] = False
    captured = list(clock["recorded"][-12:])
    for step in (2.0, 5.0):  # two replays: each re-records the captured events with new times
        clock["step"] = step
        for ev in captured:
            ev.record()
        assert col.flush() is True
        snap = col.snapshots[-1]
        assert [r.transfer_ms for r in snap.per_trap] == [step, step]
        assert [r.wait_ms for r in snap.per_trap] == [step, step]
    assert len(col.snapshots) == 2  # the eager pass before the capture was dropped, not mixed in
    clock["step"] = 3.0
    _timed_pass(col)  # eager work after the replays is timed as usual
    clock["step"] = 1.0
    _timed_pass(col)  # its start publishes the previous eager pass
    assert len(col.snapshots) == 3 and col.snapshots[-1].per_trap[0].compute_ms == 3.0


def test_eager_timing_refuses_capture():
    capturing = {"on": True}
    clock = {"now": 0.0, "step": 1.0, "recorded": []}
    col = OffloadTimingCollector(["L0"], event_factory=lambda: _ClockEvent(clock), current_stream=lambda: None,
                                 synchronize=lambda: None, is_capturing=lambda: capturing["on"])
    with pytest.raises(RuntimeError, match="cuda_graph"):
        col.on_pass_start()


def test_measure_window_stores_only_sampled_passes():
    """offload_timing.py:445-449 and offload_manager.py:1439-1469: only passes inside a sample window are stored."""
    from flextensor_amd.manager import OffloadManager

    clock = {"now": 0.0, "step": 1.0, "recorded": []}
    col = OffloadTimingCollector(["L0", "L1"], event_factory=lambda: _ClockEvent(clock), current_stream=lambda: None,
                                 synchronize=lambda: None, is_capturing=lambda: False)
    mgr = OffloadManager(name="sampling")
    mgr.timing = col
    _timed_pass(col)
    _timed_pass(col)  # an open window (the default) stores the previous pass
    assert len(col.snapshots) == 1
    mgr.reset_offload_timing_sampling()  # drops what was stored and closes the window
    assert col.snapshots == []
    _timed_pass(col)  # not sampled
    clock["step"] = 2.0
    mgr.begin_offload_timing_sample()  # drops the unsampled pass under way
    _timed_pass(col)
    assert mgr.finish_offload_timing_sample(replay_generation=None) is True
    assert len(col.snapshots) == 1 and col.snapshots[0].per_trap[0].transfer_ms == 2.0
    clock["step"] = 4.0
    _timed_pass(col)  # the window closed with the sample
    assert col.flush() is False and len(col.snapshots) == 1
    mgr.begin_offload_timing_sample()
    _timed_pass(col)
    mgr.cancel_offload_timing_sample()
    assert mgr.finish_offload_timing_sample(replay_generation=None) is False and len(col.snapshots) == 1


def test_periodic_table_every_ten_passes_even_outside_the_sample_window(caplog):
    """offload_timing.py:683-736: every finished pass goes to the rolling log table, sampled or not."""
    clock = {"now": 0.0, "step": 1.0, "recorded": []}
    col = OffloadTimingCollector(["L0", "L1"], event_factory=lambda: _ClockEvent(clock), current_stream=lambda: None,
                                 synchronize=lambda: None, is_capturing=lambda: False)
    col.set_measure_window(False)
    with caplog.at_level("INFO", logger="flextensor_amd.timing"):
        for _ in range(10):
            _timed_pass(col)
        assert "offload timing" not in caplog.text  # nine finished so far
        _timed_pass(col)  # finishes the tenth
    assert caplog.text.count("offload timing (last 10 passes") == 1 and "L0" in caplog.text
    assert col.snapshots == []  # the closed window stored none of them
