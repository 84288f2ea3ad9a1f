"""Per-trap transfer / compute / wait timing and the hidden-transfer fraction.

Same records and hooks as the reference's offload timing
(offload_timing.py:31-217, 355-720):

* ``transfer_ms`` - events around the transfer submission on the transfer
  stream;
* ``compute_ms``  - compute-stream events from ``enter`` to ``exit``;
* ``wait_ms``     - compute-stream events around the readiness wait; zero
  means the transfer was fully hidden.

A pass is finalized when the next pass starts (or on ``flush``). Device
timing uses HIP events with timing enabled. :func:`hidden_fraction` is
``1 - sum(wait) / sum(transfer)``.
"""

from __future__ import annotations

import logging
import statistics
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

LOGGER = logging.getLogger(__name__)


@dataclass(frozen=True, slots=True)
class TrapTimingRecord:
    label: str
    transfer_ms: float = 0.0
    compute_ms: float = 0.0
    wait_ms: float = 0.0


@dataclass(frozen=True, slots=True)
class OffloadTimingSnapshot:
    per_trap: Sequence[TrapTimingRecord] = ()

    def __post_init__(self) -> None:
        object.__setattr__(self, "per_trap", tuple(self.per_trap))

    @property
    def total_wait_ms(self) -> float:
        return sum(r.wait_ms for r in self.per_trap)

    @property
    def total_transfer_ms(self) -> float:
        return sum(r.transfer_ms for r in self.per_trap)

    @property
    def total_compute_ms(self) -> float:
        return sum(r.compute_ms for r in self.per_trap)


def hidden_fraction(wait_ms: float, transfer_ms: float) -> float:
    """Fraction of transfer time hidden under compute: 1 - wait / transfer."""
    if transfer_ms <= 0:
        return 1.0
    return max(0.0, min(1.0, 1.0 - wait_ms / transfer_ms))


@dataclass(frozen=True, slots=True)
class TrapTimingStats:
    """One trap's statistics over a report's passes (offload_timing.py:76-117)."""

    label: str
    compute_min: float = 0.0
    compute_max: float = 0.0
    compute_avg: float = 0.0
    compute_median: float = 0.0
    compute_std: float = 0.0
    transfer_min: float = 0.0
    transfer_max: float = 0.0
    transfer_avg: float = 0.0
    transfer_median: float = 0.0
    transfer_std: float = 0.0
    wait_min: float = 0.0
    wait_max: float = 0.0
    wait_avg: float = 0.0
    wait_median: float = 0.0
    wait_std: float = 0.0

    def compute_budget_ms(self, *, conservative: bool = False) -> float:
        """The first positive of median, mean, min (``conservative``: min, median, mean), else 0."""
        order = ((self.compute_min, self.compute_median, self.compute_avg) if conservative
                 else (self.compute_median, self.compute_avg, self.compute_min))
        return next((float(v) for v in order if v and v > 0), 0.0)


def _column_stats(values: Sequence[float]) -> tuple[float, float, float, float, float]:
    """min, max, mean, median and sample standard deviation (0 below two samples)."""
    return (min(values), max(values), sum(values) / len(values), statistics.median(values),
            statistics.stdev(values) if len(values) >= 2 else 0.0)


def build_report(passes: Sequence[OffloadTimingSnapshot]) -> "OffloadTimingReport":
    """Per-trap statistics over ``passes`` (offload_timing.py:802-855).

    Traps are matched by position; their labels come from the first pass.
    """
    passes = tuple(passes)
    if not passes:
        return OffloadTimingReport()
    labels = [r.label for r in passes[0].per_trap]
    per_trap = []
    for i, label in enumerate(labels):
        rows = [p.per_trap[i] for p in passes if i < len(p.per_trap)]
        c = _column_stats([r.compute_ms for r in rows])
        t = _column_stats([r.transfer_ms for r in rows])
        w = _column_stats([r.wait_ms for r in rows])
        per_trap.append(TrapTimingStats(label, *c, *t, *w))
    return OffloadTimingReport(per_trap=per_trap, passes=passes)


@dataclass
class OffloadTimingReport:
    """Passes of a collection window and their per-trap statistics (offload_timing.py:120-217)."""

    per_trap: Sequence[TrapTimingStats] = ()
    passes: Sequence[OffloadTimingSnapshot] = ()

    def __post_init__(self) -> None:
        self.per_trap = tuple(self.per_trap)
        self.passes = tuple(self.passes)

    @property
    def num_passes(self) -> int:
        return len(self.passes)

    @property
    def total_wait_sum(self) -> float:
        return sum(s.total_wait_ms for s in self.passes)

    @property
    def total_transfer_sum(self) -> float:
        return sum(s.total_transfer_ms for s in self.passes)

    @property
    def total_compute_sum(self) -> float:
        return sum(s.total_compute_ms for s in self.passes)

    @property
    def total_wait_avg(self) -> float:
        return self.total_wait_sum / self.num_passes if self.passes else 0.0

    @property
    def total_transfer_avg(self) -> float:
        return self.total_transfer_sum / self.num_passes if self.passes else 0.0

    @property
    def total_compute_avg(self) -> float:
        return self.total_compute_sum / self.num_passes if self.passes else 0.0

    @property
    def hidden_fraction(self) -> float:
        """Share of transfer time hidden under compute over all passes: 1 - wait / transfer."""
        return hidden_fraction(self.total_wait_sum, self.total_transfer_sum)

    def table(self) -> str:
        return format_offload_timing_table(self)


def format_offload_timing_table(data: OffloadTimingSnapshot | OffloadTimingReport) -> str:
    """A text table of one pass or of a report (offload_timing.py:220-300).

    One row per trap: compute, transfer and wait milliseconds (averages and
    medians for a report). A row whose wait exceeds 0.01 ms is flagged: its
    transfer was not hidden.
    """
    if isinstance(data, OffloadTimingReport):
        stats = data.per_trap
        if not stats:
            return "No offload timing data."
        w = max(max(len(st.label) for st in stats), 5) + 2
        rule = "=" * (w + 74)
        lines = [f"Offload Timing ({data.num_passes} passes)", rule,
                 f"{'Trap':<{w}} {'Compute avg':>12} {'med':>8}  {'Transfer avg':>13} {'med':>8}  "
                 f"{'Wait avg':>9} {'med':>8}", "-" * (w + 74)]
        for st in stats:
            flag = "  <-" if st.wait_avg > 0.01 else ""
            lines.append(f"{st.label:<{w}} {st.compute_avg:>12.3f} {st.compute_median:>8.3f}  "
                         f"{st.transfer_avg:>13.3f} {st.transfer_median:>8.3f}  "
                         f"{st.wait_avg:>9.3f} {st.wait_median:>8.3f}{flag}")
        lines += ["-" * (w + 74),
                  f"{'Avg/pass':<{w}} {data.total_compute_avg:>12.3f} {'':>8}  "
                  f"{data.total_transfer_avg:>13.3f} {'':>8}  {data.total_wait_avg:>9.3f}",
                  f"{'Sum (all)':<{w}} {data.total_compute_sum:>12.1f} {'':>8}  "
                  f"{data.total_transfer_sum:>13.1f} {'':>8}  {data.total_wait_sum:>9.1f}",
                  f"hidden fraction {data.hidden_fraction:.4f}", rule]
        return "\n".join(lines)
    if not data.per_trap:
        return "No offload timing data."
    w = max(max(len(r.label) for r in data.per_trap), 5) + 2
    rule = "=" * (w + 46)
    lines = ["Offload Timing (single pass)", rule,
             f"{'Trap':<{w}} {'Compute (ms)':>13} {'Transfer (ms)':>14} {'Wait (ms)':>10}", "-" * (w + 46)]
    for r in data.per_trap:
        flag = "  <-" if r.wait_ms > 0.01 else ""
        lines.append(f"{r.label:<{w}} {r.compute_ms:>13.3f} {r.transfer_ms:>14.3f} {r.wait_ms:>10.3f}{flag}")
    lines += ["-" * (w + 46),
              f"{'Total':<{w}} {data.total_compute_ms:>13.3f} {data.total_transfer_ms:>14.3f} "
              f"{data.total_wait_ms:>10.3f}", rule]
    return "\n".join(lines)


OFFLOAD_TIMING_LOG_EVERY = 10  # passes per periodic timing table (offload_timing.py:26)
OFFLOAD_TIMING_MEASURE_MAX_PASSES = 1024  # stored passes kept for collect_offload_timing (offload_timing.py:27)


class OffloadTimingCollector:
    """Records per-trap events during a pass; a no-op when ``enabled`` is False.

    ``event_factory()`` returns an object with ``record(stream)`` and
    ``elapsed_time(end)``; ``current_stream()`` returns the compute stream;
    ``synchronize()`` waits for the device before events are read.
    """

    def __init__(
        self,
        trap_labels: Sequence[str] | None = None,
        *,
        enabled: bool = True,
        event_factory: Callable[[], Any] | None = None,
        current_stream: Callable[[], Any] | None = None,
        synchronize: Callable[[], None] | None = None,
        on_pass: Callable[[OffloadTimingSnapshot], None] | None = None,
        max_passes: int = OFFLOAD_TIMING_MEASURE_MAX_PASSES,
        graph_replay: bool = False,
        is_capturing: Callable[[], bool] | None = None,
        log_every: int = OFFLOAD_TIMING_LOG_EVERY,
    ) -> None:
        """``graph_replay``: timing points are device timestamps written by
        kernels, so a captured pass is re-timed by every replay and
        :meth:`report` after a replay reads that replay (the role of the
        reference's external events, offload_timing.py:319-352). Read only
        after a replay: before the first one the slots hold no captured times."""
        self.enabled = enabled
        self.graph_replay = graph_replay
        self._in_capture = False
        self._capture_done: dict[str, set[str]] | None = None
        self._labels = list(trap_labels or [])
        self._label_set = set(self._labels) if enabled else set()
        self._on_pass = on_pass
        self._max_passes = max_passes
        self.snapshots: list[OffloadTimingSnapshot] = []
        self._measure_window = True  # passes are published while open (offload_timing.py:445-449)
        self._log_every = log_every
        self._log_window: list[OffloadTimingSnapshot] = []  # every finished pass, for the periodic table
        self._pass_active = False
        self._events: dict[str, dict[str, Any]] = {}
        self._done: dict[str, set[str]] = {"transfer": set(), "compute": set(), "wait": set()}
        if not enabled:
            return
        self._clock = None
        if event_factory is None or current_stream is None or synchronize is None or is_capturing is None:
            from . import hip

            if event_factory is None and graph_replay:
                # timestamps written by kernels: a captured pass is re-timed by every replay
                self._clock = hip.DeviceClock(6 * len(self._labels))
                event_factory = self._clock.event
            event_factory = event_factory or (lambda: hip.HipEvent(timing=True))
            current_stream = current_stream or hip.current_stream
            synchronize = synchronize or (lambda: hip.nat.call("ftx_device_synchronize"))
            is_capturing = is_capturing or hip.is_capturing
        self._current_stream = current_stream
        self._synchronize = synchronize
        self._is_capturing = is_capturing
        for label in self._labels:
            self._events[label] = {k: event_factory() for k in ("ts", "te", "cs", "ce", "ws", "we")}

    def set_measure_window(self, enabled: bool) -> None:
        """Publish finished passes only while the window is open (it is open from the start).

        Opening it drops an eager pass already under way, which began
        outside the window (offload_timing.py:445-449).
        """
        if enabled and not self._measure_window and self._pass_active and not self._in_capture:
            for s in self._done.values():
                s.clear()
            self._pass_active = False
        self._measure_window = enabled

    def _rec(self, label: str, key: str, stream: Any = None) -> None:
        self._events[label][key].record(stream if stream is not None else self._current_stream())

    def record_transfer_start(self, label: str, stream: Any) -> None:
        if label in self._label_set:
            self._rec(label, "ts", stream)
            self._done["transfer"].discard(label)

    def record_transfer_end(self, label: str, stream: Any) -> None:
        if label in self._label_set:
            self._rec(label, "te", stream)
            self._done["transfer"].add(label)

    def record_compute_start(self, label: str) -> None:
        if label in self._label_set:
            self._rec(label, "cs")
            self._done["compute"].discard(label)

    def record_compute_end(self, label: str) -> None:
        if label in self._label_set:
            self._rec(label, "ce")
            self._done["compute"].add(label)

    def record_wait_start(self, label: str) -> None:
        if label in self._label_set:
            self._rec(label, "ws")
            self._done["wait"].discard(label)

    def record_wait_end(self, label: str) -> None:
        if label in self._label_set:
            self._rec(label, "we")
            self._done["wait"].add(label)

    def on_pass_start(self) -> None:
        if not self.enabled:
            return
        if self._is_capturing():
            if not self.graph_replay:
                raise RuntimeError("offload_timing='eager' cannot time a captured graph; use 'cuda_graph'")
            # events are only read after a replay; a pending eager pass is dropped
            for s in self._done.values():
                s.clear()
            self._pass_active = True
            self._in_capture = True
            return
        self._end_capture()
        if self._pass_active:
            self._finalize()
        self._pass_active = True

    def _end_capture(self) -> None:
        """After a capture: keep which events the captured pass records, for reading replays."""
        if self._in_capture and not self._is_capturing():
            self._capture_done = {k: set(v) for k, v in self._done.items()}
            for s in self._done.values():
                s.clear()
            self._in_capture = False
            self._pass_active = False

    def flush(self) -> bool:
        """Publish a pending pass (the newest pass is otherwise only finalized by the next one).

        With no eager pass pending after a graph was captured, the events of
        the latest replay are read instead. Returns whether a pass was
        published (a closed measure window publishes nothing).
        """
        if not self.enabled or self._is_capturing():
            return False
        self._end_capture()
        if self._pass_active:
            return self._finalize()
        if self._capture_done is not None:
            return self._finalize(self._capture_done)
        return False

    def _finalize(self, done: dict[str, set[str]] | None = None) -> bool:
        self._synchronize()
        if self._clock is not None:
            self._clock.refresh()
        done = self._done if done is None else done
        recs = []
        for label in self._labels:
            ev = self._events[label]
            t = ev["ts"].elapsed_time(ev["te"]) if label in done["transfer"] else 0.0
            c = ev["cs"].elapsed_time(ev["ce"]) if label in done["compute"] else 0.0
            w = ev["ws"].elapsed_time(ev["we"]) if label in done["wait"] else 0.0
            recs.append(TrapTimingRecord(label, t, c, w))
        for s in self._done.values():
            s.clear()
        self._pass_active = False
        snap = OffloadTimingSnapshot(recs)
        self._maybe_log(snap)
        if not self._measure_window:
            return False
        self.snapshots.append(snap)
        del self.snapshots[: max(0, len(self.snapshots) - self._max_passes)]
        if self._on_pass is not None:
            self._on_pass(snap)
        return True

    def _maybe_log(self, snap: OffloadTimingSnapshot) -> None:
        """Every ``log_every`` finished passes, log their table at INFO (offload_timing.py:721-736)."""
        if self._log_every <= 0:
            return
        self._log_window.append(snap)
        if len(self._log_window) < self._log_every:
            return
        rep = build_report(self._log_window)
        LOGGER.info("offload timing (last %d passes, average stall per pass %.2f ms)\n%s", rep.num_passes,
                    rep.total_wait_avg, format_offload_timing_table(rep))
        self._log_window = []

    def report(self) -> OffloadTimingReport:
        self.flush()
        return build_report(self.snapshots)

    def reset(self) -> None:
        """Drop published passes and a pending eager pass; a captured pass stays readable after replays."""
        self.snapshots.clear()
        if self._in_capture:
            return  # _done holds what the captured pass records
        for s in self._done.values():
            s.clear()
        self._pass_active = False
