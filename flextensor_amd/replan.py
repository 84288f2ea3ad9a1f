"""Re-measuring a streaming plan in flight: ``request_strategy_replan`` and ``StrategyReplanStatus``.

The reference re-measures its units after an external ``torch.compile`` or a
graph capture and rebuilds its offload strategy from the new times
(offload_manager.py:1294-1325, 667-720; compile/replan_status.py). In this
build the slot plan does not depend on compute times. What does is the copy
engine of the ring: a pass whose compute is well under its time on the link
copies every ring slot with the zero-copy kernel, any other pass keeps the
per-size policy (``link_model.is_link_bound``). A replan here therefore
re-measures every unit's compute over live streamed passes (a warm-up pass,
then measured passes), stores the new times as the units' durations, and
re-decides the ring's copy policy from them.

The status snapshot keeps the reference's vocabulary: ``state`` is "idle"
before any request, "in_progress" while the passes run, "done" once they
finished (``applied`` True when the policy was rebuilt from the new times,
False when nothing in the plan depends on them) and "failed" when the rebuild
raised.
"""

from __future__ import annotations

import statistics
from collections.abc import Sequence
from dataclasses import dataclass, replace
from typing import Literal

from .link_model import LinkMeasurement, choose_copy_policy, is_link_bound
from .timing import OffloadTimingSnapshot

StrategyReplanState = Literal["idle", "in_progress", "done", "failed"]

REPLAN_WARMUP_PASSES = 1  # the first pass after a request runs with the new timing, unmeasured
REPLAN_MEASURE_PASSES = 2  # passes whose per-unit compute is measured; each unit takes the median


@dataclass(frozen=True, slots=True)
class StrategyReplanStatus:
    """Passive snapshot of a manager's replan (compile/replan_status.py:14-40); reading it changes nothing.

    ``state``: "idle" before any request, "in_progress" while the passes run,
    "done" once they finished, "failed" when the rebuild raised.
    ``can_request``: whether ``request_strategy_replan()`` would start a
    replan now. ``applied``: None before and during a request, True once the
    copy policy was rebuilt from the new times, False when the plan was kept
    (nothing measured, or nothing in the plan depends on compute times) or
    the rebuild failed.
    """

    state: StrategyReplanState
    can_request: bool
    applied: bool | None


def measured_compute(passes: Sequence[OffloadTimingSnapshot], labels: Sequence[str]) -> dict[str, float]:
    """Per unit, the median compute milliseconds over ``passes``; units no pass timed are left out."""
    out: dict[str, float] = {}
    wanted = set(labels)
    per: dict[str, list[float]] = {}
    for snap in passes:
        for rec in snap.per_trap:
            if rec.label in wanted and rec.compute_ms > 0.0:
                per.setdefault(rec.label, []).append(rec.compute_ms)
    for label in labels:
        if per.get(label):
            out[label] = float(statistics.median(per[label]))
    return out


def replanned_link(link: LinkMeasurement, compute_ms: float, streamed_sizes: Sequence[int]) -> LinkMeasurement:
    """The copy policy for a pass that computes for ``compute_ms`` and streams ``streamed_sizes``.

    The per-size policy is re-derived from the measured curves (as at the
    INFERENCE transition), then replaced by the link-bound one when the pass
    is link-bound. The curves stay the link model.
    """
    km, sm, ns = choose_copy_policy(link.sdma, link.kernel)
    transfer_ms = link.transfer_ms(list(streamed_sizes))
    base = replace(link, kernel_max_bytes=km, split_min_bytes=sm, n_copy_streams=ns, kernel_grid=0,
                   link_bound=False, pass_compute_ms=compute_ms, pass_transfer_ms=transfer_ms, source="replan")
    if streamed_sizes and is_link_bound(compute_ms, transfer_ms):
        return base.for_link_bound_pass(max(streamed_sizes))
    return base
