"""Oracle: log-log size <-> duration interpolation (memory_transfer_interpolator.py:10-183).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math


def _fit(points):
    pairs = sorted(points.items())
    xs = [math.log(float(b)) for b, _ in pairs]
    ys = [math.log(float(d)) for _, d in pairs]
    return pairs, xs, ys


def _piecewise(x, xs, ys):
    """Linear interpolation on sorted xs; end segments extended (memory_transfer_interpolator.py:76-86)."""
    if x < xs[0]:
        return ys[0] + (ys[1] - ys[0]) / (xs[1] - xs[0]) * (x - xs[0])
    if x > xs[-1]:
        return ys[-1] + (ys[-1] - ys[-2]) / (xs[-1] - xs[-2]) * (x - xs[-1])
    for i in range(1, len(xs)):
        if x <= xs[i]:
            if xs[i] == xs[i - 1]:
                return ys[i]
            t = (x - xs[i - 1]) / (xs[i] - xs[i - 1])
            return ys[i - 1] + t * (ys[i] - ys[i - 1])
    return ys[-1]


def bytes_to_duration(points, size_bytes):
    if size_bytes <= 0:
        raise ValueError(f"size_bytes must be positive, got {size_bytes}")
    pairs, xs, ys = _fit(points)
    if len(pairs) == 1:
        return float(pairs[0][1])
    return math.exp(_piecewise(math.log(float(size_bytes)), xs, ys))


def duration_to_bytes(points, duration_ms):
    """Inverse map over the duration axis (memory_transfer_interpolator.py:91-136)."""
    if duration_ms <= 0:
        raise ValueError(f"duration_ms must be positive, got {duration_ms}")
    pairs, xs, ys = _fit(points)
    if len(pairs) == 1:
        return float(pairs[0][0])
    y = math.log(float(duration_ms))
    if y < ys[0]:
        d = ys[1] - ys[0]
        return math.exp(xs[0] + ((xs[1] - xs[0]) / d) * (y - ys[0]) if d != 0 else xs[0])
    if y > ys[-1]:
        d = ys[-1] - ys[-2]
        return math.exp(xs[-1] + ((xs[-1] - xs[-2]) / d) * (y - ys[-1]) if d != 0 else xs[-1])
    return math.exp(_piecewise(y, ys, xs))


def bandwidth_mbps(points):
    """MiB/s of the largest transfer (memory_transfer_interpolator.py:138-150)."""
    b, d = max(points.items())
    return (b / (1024 * 1024)) / (d / 1000.0)
