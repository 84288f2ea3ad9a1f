"""Host-link model: live H2D measurements and a size <-> duration interpolator.

* :class:`MemoryTransferInterpolator` keeps the reference's contract
  (memory_transfer_interpolator.py:10-183): linear interpolation in log-log
  space, linear extrapolation with the slope of the two end points, and a
  constant answer when only one point is known.
* :func:`benchmark_memory_transfers` plays the role of the reference's live
  curve (memory_transfer_benchmark.py:59-129): the largest label size halved
  ``max_depth`` times, timed from pinned memory.
* :func:`measure_copy_curve` / :func:`choose_copy_policy` measure each copy
  engine of this build (SDMA, SDMA split over copy streams, zero-copy
  kernel) and derive the per-chunk-size choice the library applies under
  ``FTX_COPY_AUTO``.
* :func:`measure_link` is what the offload manager runs at the INFERENCE
  transition: both engines over log-spaced sizes up to the largest streamed
  unit, the policy they choose, and the SDMA curve in the reference's
  ``{bytes: ms}`` form (its ``memory_transfer_stats``).
* :func:`is_link_bound` then compares the profiled compute of a pass with
  the curve's time for its streamed units; a link-bound pass copies every
  ring slot with the zero-copy kernel
  (:meth:`LinkMeasurement.for_link_bound_pass`).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np

from . import _native as nat


class MemoryTransferInterpolator:
    """Bidirectional size (bytes) <-> duration (ms) model of the host link."""

    def __init__(self, memory_transfers: dict[int, float]) -> None:
        if not memory_transfers:
            raise ValueError("memory_transfers dictionary cannot be empty")
        pairs = sorted(memory_transfers.items())
        self.bytes_array = np.array([p[0] for p in pairs], dtype=np.float64)
        self.duration_array = np.array([p[1] for p in pairs], dtype=np.float64)
        if (self.bytes_array <= 0).any():
            raise ValueError("All byte values must be positive")
        if (self.duration_array <= 0).any():
            raise ValueError("All duration values must be positive")
        self.min_bytes = self.bytes_array[0]
        self.max_bytes = self.bytes_array[-1]
        self.min_duration = self.duration_array[0]
        self.max_duration = self.duration_array[-1]
        self._lx = np.log(self.bytes_array)
        self._ly = np.log(self.duration_array)
        # keep the reference's attribute names for callers that read them
        self.log_bytes = self._lx
        self.log_duration = self._ly

    @staticmethod
    def _loglog(x: float, xs: np.ndarray, ys: np.ndarray, flat_if_no_slope: bool) -> float:
        if x < xs[0]:
            i0, i1, anchor = 0, 1, 0
        elif x > xs[-1]:
            i0, i1, anchor = -2, -1, -1
        else:
            return float(np.interp(x, xs, ys))
        dx = xs[i1] - xs[i0]
        if dx == 0:
            if flat_if_no_slope:
                return float(ys[anchor])
            raise ZeroDivisionError("two points with the same abscissa")
        return float(ys[anchor] + (ys[i1] - ys[i0]) / dx * (x - xs[anchor]))

    def bytes_to_duration(self, size_bytes: int | float) -> float:
        if size_bytes <= 0:
            raise ValueError(f"size_bytes must be positive, got {size_bytes}")
        if len(self._lx) == 1:
            return float(self.duration_array[0])
        return math.exp(self._loglog(math.log(float(size_bytes)), self._lx, self._ly, False))

    def duration_to_bytes(self, duration_ms: float) -> float:
        if duration_ms <= 0:
            raise ValueError(f"duration_ms must be positive, got {duration_ms}")
        if len(self._ly) == 1:
            return float(self.bytes_array[0])
        # durations need not be sorted when measured noise is large; the
        # reference interpolates over the duration axis in byte order too.
        return math.exp(self._loglog(math.log(float(duration_ms)), self._ly, self._lx, True))

    def get_bandwidth_mbps(self) -> float:
        """MB/s (MiB-based) of the largest measured transfer."""
        return float(self.bytes_array[-1] / (1024 * 1024) / (self.duration_array[-1] / 1000.0))

    def __repr__(self) -> str:
        return (
            f"MemoryTransferInterpolator(bytes_range=[{self.min_bytes:.0f}, {self.max_bytes:.0f}], "
            f"duration_range=[{self.min_duration:.2f}, {self.max_duration:.2f}] ms, "
            f"bandwidth≈{self.get_bandwidth_mbps():.2f} MB/s)"
        )


def _human_bytes(n: int) -> str:
    for unit, scale in (("GiB", 1 << 30), ("MiB", 1 << 20), ("KiB", 1 << 10)):
        if n >= scale:
            return f"{n / scale:.1f} {unit}"
    return f"{n} B"


def format_memory_transfer_table(memory_stats: dict[int, float]) -> str:
    """The measured link curve ``{bytes: ms}`` as the diagnostic table of the reference
    (memory_transfer_benchmark.py:26-56): a rule of ``=``, the title, the rule, column
    headings, a rule of ``-``, one row per size in ascending order (bytes, the size in
    binary units, milliseconds, GB/s) and a closing ``=`` rule."""
    if not memory_stats:
        return "No memory transfer statistics available."
    rule = "=" * 110
    out = [rule, "Memory Transfer Statistics", rule,
           f"{'Size (bytes)':>14} {'Size':>10} {'Transfer (ms)':>14} {'Bandwidth (GB/s)':>17}", "-" * 110]
    for n, ms in sorted(memory_stats.items()):
        gbps = n / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        out.append(f"{n:>14} {_human_bytes(n):>10} {ms:>14.3f} {gbps:>17.3f}")
    out.append(rule)
    return "\n".join(out)


def create_interpolator_from_benchmarks(memory_transfers: dict[int, float]) -> MemoryTransferInterpolator:
    return MemoryTransferInterpolator(memory_transfers)


@dataclass
class CopyCurve:
    """Best-of-N milliseconds per size for one copy engine."""

    engine: str
    best_ms: dict[int, float] = field(default_factory=dict)

    def gbps(self) -> dict[int, float]:
        return {n: n / (ms * 1e-3) / 1e9 for n, ms in self.best_ms.items()}

    def peak_gbps(self) -> float:
        return max(self.gbps().values()) if self.best_ms else 0.0


def time_h2d(nbytes: int, engine: str, repeats: int = 10, warmup: int = 2, device=None) -> list[float]:
    """Time ``repeats`` copies of ``nbytes`` pinned host -> device with one engine.

    Engines: ``sdma`` (one hipMemcpyAsync), ``sdma_split<k>`` (split over k
    copy streams), ``kernel`` / ``kernel_g<grid>`` (zero-copy kernel).
    Returns milliseconds per copy (device events around each copy).
    """
    import torch

    from .hip import HostArena

    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"time_h2d needs a device destination, got {device}")
    arena = HostArena(nbytes)
    arena.tensor[: min(nbytes, 1 << 20)].fill_(1)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
    try:
        return _time_copies(dst, arena.ptr, nbytes, engine, repeats, warmup, device)
    finally:
        del dst


def _time_copies(dst, src_ptr: int, nbytes: int, engine: str, repeats: int, warmup: int, device) -> list[float]:
    """Milliseconds of ``repeats`` copies of ``nbytes`` from pinned ``src_ptr`` into device tensor ``dst``."""
    from .hip import HipEvent, new_stream

    if nbytes > dst.numel():
        raise ValueError(f"copy of {nbytes} bytes into a {dst.numel()}-byte buffer")
    # Each engine is timed under a policy of its own, passed with every copy: the library default and the
    # policies of managers already streaming stay as they are.
    mode, policy = nat.COPY_SDMA, nat.copy_policy(0, 2**63 - 1, 1, 0)
    if engine.startswith("sdma_split"):
        policy = nat.copy_policy(0, 1, int(engine[len("sdma_split"):]), 0)
    elif engine.startswith("kernel"):
        mode = nat.COPY_KERNEL
        policy = nat.copy_policy(0, 2**63 - 1, 1, int(engine[len("kernel_g"):]) if engine.startswith("kernel_g") else 0)
    elif engine != "sdma":
        raise ValueError(f"unknown engine {engine!r}")
    stream = new_stream(device, name="link-probe")
    try:
        times = []
        for i in range(warmup + repeats):
            e0, e1 = HipEvent(timing=True), HipEvent(timing=True)
            stream.record_event(e0)
            nat.copy_h2d(dst.data_ptr(), src_ptr, nbytes, mode, stream.handle, policy)
            stream.record_event(e1)
            e1.synchronize()
            if i >= warmup:
                times.append(e0.elapsed_time(e1))
        return times
    finally:
        stream.synchronize()


def measure_copy_curve(engine: str, sizes: list[int], repeats: int = 10, device=None) -> CopyCurve:
    curve = CopyCurve(engine)
    for n in sizes:
        curve.best_ms[n] = min(time_h2d(n, engine, repeats=repeats, device=device))
    return curve


def choose_copy_policy(sdma: CopyCurve, kernel: CopyCurve, split: CopyCurve | None = None,
                       n_split: int = 1, min_kernel_gain: float = 1.10) -> tuple[int, int, int]:
    """Per-chunk choice from measured curves.

    Returns ``(kernel_max_bytes, split_min_bytes, n_copy_streams)``: chunks up
    to ``kernel_max_bytes`` go to the zero-copy kernel, SDMA copies from
    ``split_min_bytes`` up are split over ``n_copy_streams``.

    The kernel is chosen only where it is at least ``min_kernel_gain`` times
    faster than SDMA: while it runs, its host reads hold up the memory
    accesses of kernels sharing its CUs, a cost SDMA does not have, so a few
    percent of link speed does not pay for it.
    """
    kernel_max = 0
    for n in sorted(sdma.best_ms):
        if n in kernel.best_ms and kernel.best_ms[n] * min_kernel_gain <= sdma.best_ms[n]:
            kernel_max = n
        else:
            break
    split_min = 2**63 - 1
    if split is not None and n_split > 1:
        for n in sorted(sdma.best_ms, reverse=True):
            if n in split.best_ms and split.best_ms[n] < sdma.best_ms[n]:
                split_min = n
            else:
                break
    return kernel_max, split_min, (n_split if split_min < 2**63 - 1 else 1)


# A pass whose profiled compute takes less than this share of the time its
# streamed units need on the link is link-bound: the compute stream waits on
# the link whatever runs beside it. The share leaves room for compute that
# runs slower beside the zero-copy kernel: the decode's HBM-bound GEMVs once
# ran 2.5 times longer there, before small copy grids reserved their CUs.
LINK_BOUND_COMPUTE_SHARE = 0.4
# Zero-copy kernel workgroups for the ring copies of a link-bound pass. Eight
# hold the link at its peak (57.3 GB/s for 512 MiB, against 57.1 at 64) and
# leave the compute kernels most of the chip.
RING_KERNEL_GRID = 8


def is_link_bound(compute_ms: float, transfer_ms: float, share: float = LINK_BOUND_COMPUTE_SHARE) -> bool:
    """Whether a pass that computes for ``compute_ms`` and streams for ``transfer_ms`` waits on the link.

    In such a pass the ring copies go to the zero-copy kernel. Between two
    SDMA copies of a streamed decode the link idles for 50-250 us, until the
    waiting compute kernel and the next copy start together; kernel copies
    in the same pass ran without that gap (7B-shape decode with 56 streamed
    units per token: 102.7 ms per token against 115.7). The kernel's cost,
    host reads that slow the kernels sharing its CUs, stays hidden while the
    compute stream waits on the link anyway. It is not hidden in a
    compute-bound pass: a diffusion step with 25 of 40 blocks streamed took
    4% longer with kernel copies, so such a pass keeps SDMA.
    """
    return transfer_ms > 0.0 and compute_ms < share * transfer_ms


# Exponent-coded transfers take about a quarter of the bytes off the link, and their decode holds 16 CUs while
# a transfer runs. While a pass's profiled compute stays under this share of its raw transfer time, the link
# still bounds the pass, or nearly, and fewer bytes shorten it; at or above it the transfers were hidden, and
# the held CUs would slow the compute.
ENCODE_COMPUTE_SHARE = 0.9


def encoding_pays(compute_ms: float, transfer_ms: float, share: float = ENCODE_COMPUTE_SHARE) -> bool:
    """Whether exponent-coded transfers shorten a pass that computes for ``compute_ms`` and streams raw
    blocks for ``transfer_ms``. A wider rule than :func:`is_link_bound`: between the two shares the ring
    keeps SDMA and the reference's waits, and its transfers are still encoded."""
    return transfer_ms > 0.0 and compute_ms < share * transfer_ms


def benchmark_memory_transfers(max_label_bytes: int, device=None, max_depth: int = 4,
                               max_size_bytes: int = 4 * 1024**3, engine: str = "sdma") -> dict[int, float]:
    """Median ms per size for sizes ``base / 2**d``, d < max_depth (pinned source).

    ``base`` is the largest label size capped at ``max_size_bytes`` and, as in
    the reference (memory_transfer_benchmark.py:92-102), sizes are multiples of
    4 bytes (the reference times fp32 tensors).
    """
    base = min(max_label_bytes, (max_size_bytes // 4) * 4)
    base = (base // 4) * 4
    out: dict[int, float] = {}
    for d in range(max_depth):
        n = (int(base / (2**d)) // 4) * 4
        if n <= 0:
            continue
        times = sorted(time_h2d(n, engine, repeats=10, warmup=5, device=device))
        out[n] = times[len(times) // 2]
    return out


LINK_PROBE_MIN_BYTES = 64 << 10
LINK_PROBE_MAX_BYTES = 256 << 20  # the link's rate has settled well below this; keeps the probe's buffers small


def link_probe_sizes(largest_unit_bytes: int) -> list[int]:
    """Sizes the INFERENCE-transition probe times: 64 KiB, then x4 up to the largest streamed unit (at most
    256 MiB), that size included. Multiples of 16 bytes, which every copy engine takes."""
    top = max(LINK_PROBE_MIN_BYTES, min(int(largest_unit_bytes), LINK_PROBE_MAX_BYTES)) // 16 * 16
    sizes, n = [], LINK_PROBE_MIN_BYTES
    while n < top:
        sizes.append(n)
        n *= 4
    return sizes + [top]


@dataclass
class LinkMeasurement:
    """The live copy curves of one device and the ``FTX_COPY_AUTO`` policy chosen from them."""

    sdma: CopyCurve
    kernel: CopyCurve
    kernel_max_bytes: int
    split_min_bytes: int
    n_copy_streams: int
    source: str = "measured"  # "measured" at the transition, "profile" when restored from a saved plan
    kernel_grid: int = 0  # zero-copy kernel workgroups; 0 is the library's default (64)
    link_bound: bool = False  # the ring copies of a link-bound pass all go to the kernel
    # what decided it: the pass's profiled compute and its streamed units' time on the curve
    pass_compute_ms: float | None = None
    pass_transfer_ms: float | None = None

    def memory_transfer_stats(self) -> dict[int, float]:
        """The SDMA curve as ``{bytes: ms}``, the reference's ``memory_transfer_stats`` form."""
        return dict(self.sdma.best_ms)

    def policy(self) -> tuple[int, int, int]:
        return self.kernel_max_bytes, self.split_min_bytes, self.n_copy_streams

    def native_policy(self) -> "nat.CopyPolicy":
        """This measurement's policy as the library's ``ftx_copy_policy``, for the controller that copies
        under it (every copy carries it; the library default is left alone)."""
        return nat.copy_policy(self.kernel_max_bytes, self.split_min_bytes, self.n_copy_streams, self.kernel_grid)

    def transfer_ms(self, sizes: list[int]) -> float:
        """Predicted SDMA time of copies of ``sizes`` bytes, interpolated from the measured curve."""
        if not self.sdma.best_ms:
            return 0.0
        interp = MemoryTransferInterpolator(self.sdma.best_ms)
        return float(sum(interp.bytes_to_duration(n) for n in sizes))

    def for_link_bound_pass(self, largest_unit_bytes: int) -> "LinkMeasurement":
        """The policy for a link-bound pass: every ring copy (up to ``largest_unit_bytes``) on the zero-copy
        kernel at :data:`RING_KERNEL_GRID` workgroups; the measured curves are kept."""
        return replace(self, kernel_max_bytes=max(self.kernel_max_bytes, int(largest_unit_bytes)),
                       kernel_grid=RING_KERNEL_GRID, link_bound=True)

    def describe(self) -> str:
        sd, kn = self.sdma.gbps(), self.kernel.gbps()
        curve = ", ".join(f"{n >> 10} KiB {sd[n]:.1f}/{kn.get(n, float('nan')):.1f}" for n in sorted(sd))
        where = (f"zero-copy kernel for chunks up to {self.kernel_max_bytes} bytes, SDMA above"
                 if self.kernel_max_bytes else "SDMA for every chunk")
        if self.kernel_grid:
            where += f" (kernel grid {self.kernel_grid})"
        if self.link_bound:
            where = "link-bound pass: " + where
        if self.pass_compute_ms is not None and self.pass_transfer_ms is not None:
            where += f"; pass compute {self.pass_compute_ms:.1f} ms against {self.pass_transfer_ms:.1f} ms on the link"
        return f"copy policy ({self.source}): {where}; GB/s SDMA/kernel by size: {curve}"

    def to_dict(self) -> dict:
        return {"kernel_max_bytes": self.kernel_max_bytes, "split_min_bytes": min(self.split_min_bytes, 2**63 - 1),
                "n_copy_streams": self.n_copy_streams, "kernel_grid": self.kernel_grid,
                "link_bound": self.link_bound, "pass_compute_ms": self.pass_compute_ms,
                "pass_transfer_ms": self.pass_transfer_ms,
                "sdma_ms": {str(n): ms for n, ms in sorted(self.sdma.best_ms.items())},
                "kernel_ms": {str(n): ms for n, ms in sorted(self.kernel.best_ms.items())}}

    @classmethod
    def from_dict(cls, data: dict, source: str = "profile") -> "LinkMeasurement":
        try:
            sdma = CopyCurve("sdma", {int(k): float(v) for k, v in data.get("sdma_ms", {}).items()})
            kernel = CopyCurve("kernel", {int(k): float(v) for k, v in data.get("kernel_ms", {}).items()})
            km, sm, ns = int(data["kernel_max_bytes"]), int(data["split_min_bytes"]), int(data["n_copy_streams"])
            kg = int(data.get("kernel_grid", 0))  # plans saved before the grid was recorded use the default
            bound = data.get("link_bound", False)
            times = [None if data.get(k) is None else float(data[k]) for k in ("pass_compute_ms", "pass_transfer_ms")]
        except (KeyError, TypeError, ValueError) as exc:
            raise ValueError(f"invalid copy_policy in the saved state: {exc}") from exc
        if km < 0 or sm < 0 or not 1 <= ns <= 8 or not 0 <= kg <= 1 << 20 or not isinstance(bound, bool) \
                or any(v <= 0 for v in sdma.best_ms.values()) or any(t is not None and t < 0 for t in times):
            raise ValueError("invalid copy_policy in the saved state: out-of-range values")
        return cls(sdma, kernel, km, sm, ns, source, kg, bound, *times)


def measure_link(sizes: list[int], device=None, repeats: int = 5, warmup: int = 1) -> LinkMeasurement:
    """Best-of-``repeats`` host-to-device ms per size for SDMA and for the zero-copy kernel, from one pinned
    arena into one device buffer of the largest size, and the policy :func:`choose_copy_policy` picks."""
    import torch

    from .hip import HostArena

    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    top = max(sizes)
    arena = HostArena(top)
    arena.tensor[: min(top, 1 << 20)].fill_(1)
    dst = torch.empty(top, dtype=torch.uint8, device=device)
    try:
        curves = {}
        for engine in ("sdma", "kernel"):
            curve = CopyCurve(engine)
            for n in sizes:
                curve.best_ms[n] = min(_time_copies(dst, arena.ptr, n, engine, repeats, warmup, device))
            curves[engine] = curve
    finally:
        del dst
    km, sm, ns = choose_copy_policy(curves["sdma"], curves["kernel"])
    return LinkMeasurement(curves["sdma"], curves["kernel"], km, sm, ns)
