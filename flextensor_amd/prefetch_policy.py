"""Detects prefetches whose wait is cut off by a graph-piece join.

Same contract as the reference's ``PiecewisePrefetchPolicy``
(piecewise_prefetch_policy.py:52-151): loaders call the hooks
unconditionally; a disabled policy is a no-op. A prefetch scheduled before a
piece join and waited after it loses its overlap (the join drains the
transfer stream), which the policy reports as a warning or, in strict mode,
as :class:`PiecewisePrefetchPolicyError`. At the end-of-forward join, pairs
whose compute label was already waited during the pass are next-pass
prefetches and are not reported.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass

LOGGER = logging.getLogger(__name__)


class PiecewisePrefetchPolicyError(RuntimeError):
    """A piece join interrupted an outstanding prefetch (strict mode)."""


@dataclass(frozen=True, slots=True)
class OutstandingPrefetch:
    schedule_label: str
    compute_label: str


class PiecewisePrefetchPolicy:
    def __init__(self, *, enabled: bool = False, strict: bool = False) -> None:
        self.enabled = enabled
        self.strict = strict
        self._outstanding: dict[str, str] = {}  # compute label -> schedule label
        self._reported: set[tuple[str, str]] = set()
        self._waited: set[str] = set()

    def reset(self) -> None:
        self._outstanding.clear()
        self._waited.clear()

    def on_schedule(self, schedule_label: str, compute_label: str) -> None:
        if self.enabled:
            self._outstanding[compute_label] = schedule_label

    def on_wait(self, compute_label: str) -> None:
        if self.enabled:
            self._outstanding.pop(compute_label, None)
            self._waited.add(compute_label)

    def on_piece_join(self, *, at_last_layer: bool = False) -> list[OutstandingPrefetch]:
        if not self.enabled:
            return []
        pending = [OutstandingPrefetch(s, c) for c, s in self._outstanding.items()]
        self._outstanding.clear()
        broken = [p for p in pending if not (at_last_layer and p.compute_label in self._waited)]
        if not broken:
            return []
        fresh = [p for p in broken if (p.schedule_label, p.compute_label) not in self._reported]
        self._reported.update((p.schedule_label, p.compute_label) for p in fresh)
        if not fresh and not self.strict:
            return broken
        pairs = ", ".join(
            repr(p.schedule_label) if p.schedule_label == p.compute_label else f"{p.schedule_label!r}→{p.compute_label!r}"
            for p in (fresh or broken)
        )
        where = "end-of-forward join" if at_last_layer else "PIECEWISE piece join"
        msg = (
            f"piecewise prefetch policy: {where} with outstanding H2D prefetch(es) [{pairs}]; "
            "the join forced these transfers to finish before their waits, so their overlap is lost"
        )
        if self.strict:
            raise PiecewisePrefetchPolicyError(msg)
        LOGGER.warning(msg)
        return broken
