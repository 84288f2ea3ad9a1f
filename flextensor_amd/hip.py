"""Streams, events and host arenas over the C ABI.

:class:`HipStream` wraps a ``hipStream_t`` (normally the handle of a
``torch.cuda.Stream``) and offers the ``record_event / wait_event /
wait_stream / synchronize`` surface the transfer runtime uses, in the
shape the reference uses PyTorch's stream objects (core/transfer.py:49-146).
:class:`HostArena` is one page-locked, device-mapped host allocation exposed
as a CPU ``uint8`` tensor without copying.
"""

from __future__ import annotations

import ctypes
from collections.abc import Iterator
from contextlib import contextmanager
from typing import Any

import torch

from . import _native as nat


_FREE_EVENTS: dict[int, list[int]] = {}  # recycled handles by creation flags
_MAX_FREE_EVENTS = 4096


class HipEvent:
    """One ``hipEvent_t``.

    Handles are recycled through a free list instead of being destroyed: the
    streaming loop creates and drops several events per label, and an event
    dropped by Python may still be pending on a stream. Re-recording a
    recycled handle is safe because a wait always refers to the record that
    preceded it.
    """

    __slots__ = ("handle", "timing", "flags", "__weakref__")

    def __init__(self, timing: bool = False, device_only: bool = False) -> None:
        """``device_only``: only streams of this device wait on it, so recording it skips the system-scope
        fence (``FTX_EVENT_DEVICE_ONLY``); host waits still see it complete."""
        self.timing = timing
        self.flags = (nat.EVENT_TIMING if timing else nat.EVENT_DEFAULT) | (nat.EVENT_DEVICE_ONLY if device_only else 0)
        free = _FREE_EVENTS.setdefault(self.flags, [])
        self.handle = free.pop() if free else nat.event_create(self.flags)

    def record(self, stream: "HipStream | None" = None) -> "HipEvent":
        s = stream if stream is not None else current_stream()
        nat.call("ftx_event_record", self.handle, s.handle)
        return self

    def query(self) -> bool:
        return nat.event_query(self.handle)

    def synchronize(self) -> None:
        nat.call("ftx_event_synchronize", self.handle)

    def elapsed_time(self, end: "HipEvent") -> float:
        return nat.event_elapsed_ms(self.handle, end.handle)

    def __del__(self) -> None:
        h = getattr(self, "handle", None)
        if not h:
            return
        self.handle = None
        try:
            if not nat.live():
                return
            free = _FREE_EVENTS.setdefault(self.flags, [])
            if len(free) < _MAX_FREE_EVENTS:
                free.append(h)
            else:
                nat.lib().ftx_event_destroy(h)
        except (TypeError, AttributeError):
            pass  # interpreter shutdown: module globals are already gone; the process frees the handle


class DeviceClock:
    """A device array of wall-clock timestamps written by ``ftx_timestamp``.

    Its events are kernel launches, so a graph that captures them writes new
    times on every replay. :meth:`refresh` copies the array to the host once
    the device is idle; elapsed times are then read from that copy.
    """

    def __init__(self, n: int, device: torch.device | int | None = None) -> None:
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.buf = torch.zeros(max(1, n), dtype=torch.int64, device=dev)
        self.host: list[int] = [0] * max(1, n)
        khz = ctypes.c_int(0)
        nat.call("ftx_wall_clock_khz", ctypes.byref(khz))
        if khz.value <= 0:
            raise RuntimeError("the device reports no wall-clock rate")
        self.ticks_per_ms = float(khz.value)
        self._next = 0

    def event(self) -> "ClockEvent":
        if self._next >= self.buf.numel():
            raise RuntimeError(f"device clock has only {self.buf.numel()} slots")
        self._next += 1
        return ClockEvent(self, self._next - 1)

    def refresh(self) -> None:
        self.host = self.buf.cpu().tolist()


class ClockEvent:
    """One timestamp slot of a :class:`DeviceClock`, with the ``record`` / ``elapsed_time`` of an event."""

    __slots__ = ("clock", "index")

    def __init__(self, clock: DeviceClock, index: int) -> None:
        self.clock, self.index = clock, index

    def record(self, stream: "HipStream | None" = None) -> "ClockEvent":
        s = stream if stream is not None else current_stream()
        nat.call("ftx_timestamp", self.clock.buf.data_ptr() + 8 * self.index, s.handle)
        return self

    def elapsed_time(self, end: "ClockEvent") -> float:
        h = self.clock.host
        return (h[end.index] - h[self.index]) / self.clock.ticks_per_ms


class HipStream:
    """A HIP stream. ``torch_stream`` keeps the owning torch object alive."""

    __slots__ = ("handle", "torch_stream", "name", "__weakref__")

    def __init__(self, torch_stream: Any = None, handle: int | None = None, name: str = "") -> None:
        self.torch_stream = torch_stream
        self.handle = int(handle if handle is not None else torch_stream.cuda_stream)
        self.name = name

    def record_event(self, event: HipEvent | None = None) -> HipEvent:
        return (event if event is not None else HipEvent()).record(self)

    def wait_event(self, event: HipEvent) -> None:
        nat.call("ftx_stream_wait_event", self.handle, event.handle)

    def wait_stream(self, other: "HipStream") -> None:
        self.wait_event(other.record_event())

    def synchronize(self) -> None:
        nat.call("ftx_stream_synchronize", self.handle)

    def query(self) -> bool:
        done = ctypes.c_int(0)
        nat.call("ftx_stream_query", self.handle, ctypes.byref(done))
        return bool(done.value)

    def __eq__(self, other: object) -> bool:
        return isinstance(other, HipStream) and other.handle == self.handle

    def __hash__(self) -> int:
        return hash(self.handle)

    def __repr__(self) -> str:
        return f"HipStream({self.name or hex(self.handle)})"


def is_capturing() -> bool:
    """Whether torch's current stream is capturing a graph (False without a GPU)."""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def current_stream(device: torch.device | int | None = None) -> HipStream:
    """torch's current stream on ``device`` as a :class:`HipStream`."""
    return HipStream(torch.cuda.current_stream(device), name="compute")


def new_stream(device: torch.device | int | None = None, name: str = "transfer") -> HipStream:
    """A new stream at default priority, owned by torch's stream pool."""
    return HipStream(torch.cuda.Stream(device=device), name=name)


_TRANSFER_STREAMS: dict[int, HipStream] = {}
_REJECTED_STREAMS: list[Any] = []  # kept alive so later streams are not handed the same queue again
_STREAM_PROBES: dict[int, dict[str, Any]] = {}


class TransferStreamError(RuntimeError):
    """No new stream ran beside the compute stream: transfers would queue behind every forward kernel."""


def _probe_concurrency(candidate: HipStream, compute: HipStream, device: torch.device) -> tuple[float, float]:
    """``(busy_ms, candidate_ms)``: how long the compute stream's queued work took, and when a tiny fill
    queued on ``candidate`` at the same time finished.

    Streams share the device's hardware queues; a stream on the compute
    stream's queue waits behind every compute packet. The probe queues about
    two milliseconds of matrix products on ``compute`` (enqueued in a tenth of
    that) and a one-kilobyte fill on ``candidate``.
    """
    a = torch.ones(4096, 4096, dtype=torch.bfloat16, device=device)
    small = torch.empty(1024, dtype=torch.uint8, device=device)
    with torch.cuda.stream(compute.torch_stream) if compute.torch_stream is not None else _nullctx():
        torch.matmul(a, a)  # the first product at a shape selects its kernel on the host: keep that out of the window
    torch.cuda.synchronize(device)
    c_end, s_end, start = HipEvent(timing=True), HipEvent(timing=True), HipEvent(timing=True)
    compute.record_event(start)
    with torch.cuda.stream(compute.torch_stream) if compute.torch_stream is not None else _nullctx():
        for _ in range(16):
            torch.matmul(a, a)
    compute.record_event(c_end)
    with torch.cuda.stream(candidate.torch_stream):
        small.fill_(1)
    candidate.record_event(s_end)
    torch.cuda.synchronize(device)
    return start.elapsed_time(c_end), start.elapsed_time(s_end)


# A candidate on the compute stream's hardware queue finishes its fill only after all of the queued
# products (at about 100% of the busy time); one on another queue finishes within the first half, or
# around 60% when a profiler's tracing slows every dispatch. 80% separates the two.
_CONCURRENT_FRACTION = 0.8


def _runs_concurrently(candidate: HipStream, compute: HipStream, device: torch.device) -> bool:
    """Whether work on ``candidate`` finishes while ``compute`` is still busy."""
    busy, cand = _probe_concurrency(candidate, compute, device)
    return cand < _CONCURRENT_FRACTION * busy


def transfer_stream(device: torch.device | int | None = None, attempts: int = 8) -> HipStream:
    """The per-device stream used for host-to-device transfers.

    Chosen once per device among new default-priority streams: the first one
    whose work runs concurrently with torch's current stream (see
    :func:`_probe_concurrency`). Rejected candidates stay allocated, so the
    pool does not hand their queue out again. If none of ``attempts``
    candidates runs beside the compute stream, :class:`TransferStreamError`
    names the measurements. :func:`transfer_stream_probe` reports the outcome.
    """
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    cached = _TRANSFER_STREAMS.get(dev.index)
    if cached is not None:
        return cached
    compute = current_stream(dev)
    tried: list[tuple[float, float]] = []
    for i in range(attempts):
        cand = new_stream(dev, name="transfer")
        busy, done = _probe_concurrency(cand, compute, dev)
        tried.append((round(busy, 3), round(done, 3)))
        if done < _CONCURRENT_FRACTION * busy:
            _STREAM_PROBES[dev.index] = {"chosen_candidate": i, "rejected": i, "attempts": attempts,
                                         "compute_busy_ms": tried[-1][0], "transfer_fill_done_ms": tried[-1][1]}
            _TRANSFER_STREAMS[dev.index] = cand
            return cand
        _REJECTED_STREAMS.append(cand)
    raise TransferStreamError(
        f"no transfer stream on cuda:{dev.index} runs beside the compute stream: each of {attempts} new "
        f"default-priority streams finished a 1 KB fill only after the compute stream's queued matrix products "
        f"(compute busy ms, fill done ms per candidate: {tried}). Every candidate shares the compute stream's "
        "hardware queue, so transfers would wait behind each forward kernel; check GPU_MAX_HW_QUEUES and other "
        "work on this device")


def transfer_stream_probe(device: torch.device | int | None = None) -> dict[str, Any] | None:
    """How the transfer stream of ``device`` was chosen: candidate index, rejected count and the timings
    of the accepted probe; None before :func:`transfer_stream` ran there."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    return _STREAM_PROBES.get(dev.index if dev.index is not None else torch.cuda.current_device())


@contextmanager
def use_stream(stream: HipStream) -> Iterator[None]:
    """Make ``stream`` torch's current stream inside the block."""
    if stream.torch_stream is None:
        raise ValueError("use_stream needs a stream created through torch")
    with torch.cuda.stream(stream.torch_stream):
        yield


class _ArenaOwner:
    """Frees one arena when the last reference to it goes away."""

    __slots__ = ("ptr",)

    def __init__(self, ptr: int) -> None:
        self.ptr = ptr

    def __del__(self) -> None:
        ptr, self.ptr = self.ptr, 0
        if not ptr:
            return
        try:
            if nat.live():
                nat.lib().ftx_arena_free(ptr)
        except (TypeError, AttributeError):
            pass  # interpreter shutdown: module globals are already gone; the process frees the arena


class HostArena:
    """Page-locked, device-mapped host bytes from ``ftx_arena_alloc``.

    ``tensor`` is a CPU ``uint8`` tensor over the arena. Ownership runs one
    way - tensor -> buffer -> owner - so the memory is returned by reference
    counting as soon as this object and every view of the tensor are gone
    (no cycle waits for the garbage collector while pinned memory is held).
    """

    def __init__(self, nbytes: int, flags: int = nat.ARENA_DEFAULT) -> None:
        if nbytes <= 0:
            raise ValueError(f"arena size must be positive, got {nbytes}")
        self.nbytes = int(nbytes)
        self.flags = flags
        self.ptr = nat.arena_alloc(self.nbytes, flags)
        owner = _ArenaOwner(self.ptr)
        self.device_ptr = nat.host_device_ptr(self.ptr)
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        buf._ftx_owner = owner  # every view holds the buffer, the buffer holds the owner
        self.tensor = torch.frombuffer(buf, dtype=torch.uint8)


def copy_h2d(dst: torch.Tensor, src: torch.Tensor, mode: int, stream: HipStream | None = None,
             nbytes: int | None = None, policy: nat.CopyPolicy | None = None) -> None:
    """Stream-ordered copy of ``nbytes`` (default: all of ``src``) host -> device, under ``policy`` (None: the
    library default)."""
    n = src.numel() * src.element_size() if nbytes is None else int(nbytes)
    if n > dst.numel() * dst.element_size():
        raise ValueError(f"copy of {n} bytes does not fit destination of {dst.numel() * dst.element_size()} bytes")
    if src.device.type != "cpu" or dst.device.type != "cuda":
        raise ValueError("copy_h2d needs a CPU source and a device destination")
    s = stream if stream is not None else current_stream(dst.device)
    nat.copy_h2d(dst.data_ptr(), src.data_ptr(), n, mode, s.handle, policy)


def checksum(t: torch.Tensor, stream: HipStream | None = None) -> int:
    """Device checksum of the bytes of a contiguous device tensor."""
    if t.device.type != "cuda" or not t.is_contiguous():
        raise ValueError("checksum needs a contiguous device tensor")
    s = stream if stream is not None else current_stream(t.device)
    return nat.checksum64(t.data_ptr(), t.numel() * t.element_size(), s.handle)


FP8_DECODE_MAX_ROWS = 64  # more rows run the tiled prefill kernel
_FP8_WORKSPACE: dict[tuple, int] = {}


def fp8_linear_workspace_bytes(m: int, n: int, k: int) -> int:
    """Bytes of device workspace one ``fp8_linear`` call of this shape needs (cached per shape)."""
    key = (m, n, k)
    got = _FP8_WORKSPACE.get(key)
    if got is None:
        b = ctypes.c_size_t(0)
        nat.call("ftx_fp8_linear_workspace", m, n, k, ctypes.byref(b))
        got = _FP8_WORKSPACE[key] = int(b.value)
    return got


def _check_fp8_operands(what: str, x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor) -> tuple[int, int, int]:
    """Ranks, dtypes, shapes and devices of an fp8 linear's operands; returns (m, k, n)."""
    if x.dim() != 2 or weight.dim() != 2 or scale.dim() != 1:
        raise ValueError(f"{what} needs x [m, k], weight [n, k] and scale [n]")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.float8_e4m3fn or scale.dtype != torch.bfloat16:
        raise TypeError(f"{what} needs bf16 x, float8_e4m3fn weight and bf16 scale; got "
                        f"{x.dtype}, {weight.dtype}, {scale.dtype}")
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k or scale.shape[0] != n:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, weight {tuple(weight.shape)}, scale {tuple(scale.shape)}")
    if not (x.is_cuda and weight.device == x.device and scale.device == x.device):
        raise ValueError(f"{what} needs x, weight and scale on one GPU")
    return m, k, n


def fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``bf16(scale * (x @ weight.T))`` by the library's fp8-weight MFMA kernel.

    ``x``: bf16 ``[m, k]``; ``weight``: float8 e4m3fn ``[n, k]``; ``scale``:
    bf16 ``[n]``; all on one device. The weights are widened to bf16 in
    registers, so the products are those of dequantizing and running a bf16
    GEMM. Up to 64 rows run the split-K decode kernel, more rows the tiled
    prefill kernel. Runs on torch's current stream; a split-K workspace comes
    from torch's allocator on that stream.
    """
    m, k, n = _check_fp8_operands("fp8_linear", x, weight, scale)
    if not weight.is_contiguous() or weight.data_ptr() % 16:
        raise ValueError("fp8_linear needs a contiguous, 16-byte aligned weight")
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.clone(memory_format=torch.contiguous_format)
    if not scale.is_contiguous():
        scale = scale.contiguous()
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    ws_bytes = fp8_linear_workspace_bytes(m, n, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    nat.call("ftx_fp8_linear", x.data_ptr(), weight.data_ptr(), scale.data_ptr(), y.data_ptr(), m, n, k,
             ws.data_ptr() if ws is not None else None, ws_bytes, torch.cuda.current_stream(x.device).cuda_stream)
    return y


def fp8_linear_group_workspace_bytes(m: int, ns: list[int], k: int) -> int:
    """Bytes of device workspace one ``fp8_linear_group`` call of these shapes needs (cached per shape)."""
    key = ("group", m, k) + tuple(ns)  # distinct from the (m, n, k) keys of single calls
    got = _FP8_WORKSPACE.get(key)
    if got is None:
        arr = (ctypes.c_int64 * len(ns))(*ns)
        b = ctypes.c_size_t(0)
        nat.call("ftx_fp8_linear_group_workspace", m, ctypes.cast(arr, ctypes.c_void_p), len(ns), k, ctypes.byref(b))
        got = _FP8_WORKSPACE[key] = int(b.value)
    return got


def fp8_linear_group(x: torch.Tensor, weights: list[torch.Tensor], scales: list[torch.Tensor]) -> list[torch.Tensor]:
    """``[fp8_linear(x, w, s) for w, s in zip(weights, scales)]`` in one launch (``ftx_fp8_linear_group``).

    For up to four weight matrices that share ``x`` and ``k`` (a layer's q/k/v or gate/up projections): the
    group pays one kernel launch, and one reduce launch when K is split, instead of one of each per matrix.
    Each output equals the single call's to within fp32 rounding (the group may split K differently).
    """
    if not 1 <= len(weights) <= 4 or len(weights) != len(scales):
        raise ValueError("fp8_linear_group takes 1 to 4 weights with one scale each")
    if x.dim() != 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("fp8_linear_group needs a bf16 GPU x [m, k]")
    m, k = x.shape
    for w, sc in zip(weights, scales):
        if w.dtype != torch.float8_e4m3fn or w.dim() != 2 or w.shape[1] != k or w.device != x.device:
            raise ValueError(f"every weight must be float8_e4m3fn [n, {k}] on {x.device}")
        if not w.is_contiguous() or w.data_ptr() % 16:
            raise ValueError("fp8_linear_group needs contiguous, 16-byte aligned weights")
        if sc.dtype != torch.bfloat16 or sc.shape != (w.shape[0],) or sc.device != x.device:
            raise ValueError("every scale must be bf16 [n] on the input's device")
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.clone(memory_format=torch.contiguous_format)
    scales = [sc if sc.is_contiguous() else sc.contiguous() for sc in scales]
    g = len(weights)
    ns = (ctypes.c_int64 * g)(*[w.shape[0] for w in weights])
    outs = [torch.empty((m, w.shape[0]), dtype=torch.bfloat16, device=x.device) for w in weights]
    ws_bytes = fp8_linear_group_workspace_bytes(m, list(ns), k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    ptrs = [(ctypes.c_void_p * g)(*[t.data_ptr() for t in ts]) for ts in (weights, scales, outs)]
    nat.call("ftx_fp8_linear_group", x.data_ptr(), g, *(ctypes.cast(a, ctypes.c_void_p) for a in ptrs),
             ctypes.cast(ns, ctypes.c_void_p), m, k, ws.data_ptr() if ws is not None else None, ws_bytes,
             torch.cuda.current_stream(x.device).cuda_stream)
    return outs


def fp8_linear_fused_workspace_bytes(m: int, ns: list[int], k: int, epilogue: int) -> int:
    """Bytes of device workspace one ``ftx_fp8_linear_fused`` call of these shapes needs (cached per shape)."""
    key = ("fused", epilogue, m, k) + tuple(ns)
    got = _FP8_WORKSPACE.get(key)
    if got is None:
        arr = (ctypes.c_int64 * len(ns))(*ns)
        b = ctypes.c_size_t(0)
        nat.call("ftx_fp8_linear_fused_workspace", m, ctypes.cast(arr, ctypes.c_void_p), len(ns), k, epilogue,
                 ctypes.byref(b))
        got = _FP8_WORKSPACE[key] = int(b.value)
    return got


def _fp8_fused(x: torch.Tensor, weights: list[torch.Tensor], scales: list[torch.Tensor], epilogue: int,
               residual: torch.Tensor | None, what: str) -> torch.Tensor:
    ms = [_check_fp8_operands(what, x, w, sc) for w, sc in zip(weights, scales)]
    m, k, n = ms[0]
    if m > FP8_DECODE_MAX_ROWS:
        raise ValueError(f"{what} runs in the decode kernel: at most {FP8_DECODE_MAX_ROWS} rows, got {m}")
    for w in weights:
        if not w.is_contiguous() or w.data_ptr() % 16:
            raise ValueError(f"{what} needs contiguous, 16-byte aligned weights")
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.clone(memory_format=torch.contiguous_format)
    scales = [sc if sc.is_contiguous() else sc.contiguous() for sc in scales]
    if residual is not None:
        if residual.shape != (m, n) or residual.dtype != torch.bfloat16 or residual.device != x.device:
            raise ValueError(f"{what}: the residual must be bf16 [{m}, {n}] on {x.device}")
        if not residual.is_contiguous():
            residual = residual.contiguous()
    g = len(weights)
    ns = [w.shape[0] for w in weights]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    ws_bytes = fp8_linear_fused_workspace_bytes(m, ns, k, epilogue)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    arrays = [(ctypes.c_void_p * g)(*[t.data_ptr() for t in ts]) for ts in (weights, scales)]
    n_arr = (ctypes.c_int64 * g)(*ns)
    nat.call("ftx_fp8_linear_fused", x.data_ptr(), g, *(ctypes.cast(a, ctypes.c_void_p) for a in arrays),
             y.data_ptr(), ctypes.cast(n_arr, ctypes.c_void_p), m, k, epilogue,
             residual.data_ptr() if residual is not None else None, ws.data_ptr(), ws_bytes,
             torch.cuda.current_stream(x.device).cuda_stream)
    return y


def fp8_linear_swiglu(x: torch.Tensor, w_gate: torch.Tensor, s_gate: torch.Tensor, w_up: torch.Tensor,
                      s_up: torch.Tensor) -> torch.Tensor:
    """``F.silu(g) * u`` for ``g, u = fp8_linear(x, w_gate, s_gate), fp8_linear(x, w_up, s_up)`` in one grouped
    launch plus its reduce (``FTX_FP8_EPILOGUE_SWIGLU``): a SwiGLU MLP's gate and up projections and their
    activation. Decode batches only (at most 64 rows); g and u are rounded to bf16 as the separate
    projections round them, silu(g) is rounded to bf16, then the product."""
    if w_gate.shape != w_up.shape:
        raise ValueError(f"gate and up weights differ in shape: {tuple(w_gate.shape)} and {tuple(w_up.shape)}")
    return _fp8_fused(x, [w_gate, w_up], [s_gate, s_up], nat.FP8_EPILOGUE_SWIGLU, None, "fp8_linear_swiglu")


def fp8_linear_residual(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                        residual: torch.Tensor) -> torch.Tensor:
    """``residual + fp8_linear(x, weight, scale)`` with the add folded into the reduce
    (``FTX_FP8_EPILOGUE_RESIDUAL``): a decoder's output projection and its residual connection. Decode
    batches only (at most 64 rows); the same bits as the separate linear and bf16 add."""
    return _fp8_fused(x, [weight], [scale], nat.FP8_EPILOGUE_RESIDUAL, residual, "fp8_linear_residual")


def fp8_linear_static(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``fp8_linear`` into ``out`` (bf16 ``[m, n]``) with no allocation at all, for graph capture and serving
    loops: the split-K partial sums live in the library's static per-GPU scratch array
    (``ftx_fp8_linear_static``). Operands must already be contiguous and 16-byte aligned. Calls that may
    overlap on one GPU share that scratch and must be ordered (one stream). Every operand is checked as
    ``fp8_linear`` checks it (dtypes, shapes, one device); nothing is copied to fix a layout."""
    m, k, n = _check_fp8_operands("fp8_linear_static", x, weight, scale)
    if out.shape != (m, n) or out.dtype != torch.bfloat16 or not out.is_contiguous() or out.device != x.device:
        raise ValueError(f"out must be a contiguous bf16 [{m}, {n}] tensor on {x.device}")
    for name, t in (("x", x), ("weight", weight)):
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise ValueError(f"fp8_linear_static needs a contiguous, 16-byte aligned {name}")
    if not scale.is_contiguous():
        raise ValueError("fp8_linear_static needs a contiguous scale")
    nat.call("ftx_fp8_linear_static", x.data_ptr(), weight.data_ptr(), scale.data_ptr(), out.data_ptr(), m, n, k,
             torch.cuda.current_stream(x.device).cuda_stream)
    return out


def set_fp8_linear_config(waves: int = 0, slice_k: int = 0) -> None:
    """Fix the fp8 linear launch shape: wavefronts per workgroup and K values
    per workgroup (0 = chosen per call from the shape)."""
    nat.call("ftx_set_fp8_linear_config", waves, slice_k)
    _FP8_WORKSPACE.clear()
