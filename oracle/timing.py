"""Oracle: offload-timing aggregation and the hidden-transfer fraction.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates offload_timing.py:31-117 (per-pass totals of a snapshot) and the
report builder offload_timing.py:802-855 (per-trap min / max / mean / median /
sample standard deviation, traps matched by position, labels from the first
pass), on plain tuples ``(label, transfer_ms, compute_ms, wait_ms)``. The
hidden fraction is ``1 - sum(wait) / sum(transfer)`` clipped to [0, 1]
(``wait_ms == 0`` means fully hidden: docs/how-to/configure-for-common-scenarios.md:182).
"""

from __future__ import annotations

import math


def pass_totals(records):
    """(transfer, compute, wait) sums of one pass."""
    return (math.fsum(r[1] for r in records), math.fsum(r[2] for r in records), math.fsum(r[3] for r in records))


def _median(v):
    s = sorted(v)
    n = len(s)
    return s[n // 2] if n % 2 else (s[n // 2 - 1] + s[n // 2]) / 2


def _stdev(v):
    if len(v) < 2:
        return 0.0
    m = math.fsum(v) / len(v)
    return math.sqrt(math.fsum((x - m) ** 2 for x in v) / (len(v) - 1))


def per_trap_stats(passes):
    """{label: {"compute"|"transfer"|"wait": (min, max, mean, median, stdev)}} in first-pass order."""
    if not passes:
        return {}
    out = {}
    for i, rec in enumerate(passes[0]):
        rows = [p[i] for p in passes if i < len(p)]
        cols = {"transfer": [r[1] for r in rows], "compute": [r[2] for r in rows], "wait": [r[3] for r in rows]}
        out[rec[0]] = {k: (min(v), max(v), math.fsum(v) / len(v), _median(v), _stdev(v)) for k, v in cols.items()}
    return out


def hidden_fraction(passes):
    transfer = math.fsum(pass_totals(p)[0] for p in passes)
    wait = math.fsum(pass_totals(p)[2] for p in passes)
    if transfer <= 0:
        return 1.0
    return max(0.0, min(1.0, 1.0 - wait / transfer))
