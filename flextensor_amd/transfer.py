"""Stream/event runtime that orders host-to-device transfers against slot consumers.

Contract of the reference's ``CudaTransferRuntime`` (core/transfer.py:39-146),
rebuilt on HIP streams and events through the C ABI:

* ``begin()`` forks the current (compute) stream into the transfer stream
  (:62-71);
* ``submit(slot, fn)`` rejects a busy slot (:88-89), makes the transfer stream
  wait for the slot's last use (:90-92), runs ``fn`` with the transfer stream
  current and records a readiness event (:96-100);
* ``wait_ready(ticket)`` makes the current stream wait for a live ticket and
  rejects stale or foreign tickets (:102-109). ``wait_ready(ticket, host=True)``
  blocks the calling thread on the ticket instead, so that no wait on another
  queue is pending while the transfer runs;
* ``finish_use(slot)`` records the slot's last use on the current stream
  (:111-117);
* ``join()`` joins the transfer stream back and invalidates tickets (:119-131);
* ``close()`` synchronizes once and refuses further work (:133-142).

Streams come from a :class:`StreamBackend`; :class:`HipBackend` is the device
backend, and tests inject a recording fake with the same four methods.
One host thread owns an instance; the runtime is not thread-safe.
"""

from __future__ import annotations

from collections.abc import Callable, Hashable
from contextlib import AbstractContextManager
from dataclasses import dataclass, field
from typing import Any, Protocol


class TransferStreamSynchronizationError(RuntimeError):
    """The transfer stream could not be joined or synchronized."""


def synchronize_transfer_stream(stream: Any) -> None:
    try:
        stream.synchronize()
    except Exception as error:  # noqa: BLE001 - re-raised with the runtime's error type
        raise TransferStreamSynchronizationError(str(error)) from error


class StreamBackend(Protocol):
    def current_stream(self) -> Any: ...

    def new_stream(self, device: Any) -> Any: ...

    def use_stream(self, stream: Any) -> AbstractContextManager: ...

    def is_capturing(self) -> bool: ...


class HipBackend:
    """Streams and events of the HIP runtime torch uses, through the C ABI."""

    def __init__(self, device: Any = None) -> None:
        self.device = device

    def current_stream(self) -> Any:
        from .hip import current_stream

        return current_stream(self.device)

    def new_stream(self, device: Any) -> Any:
        """The device's transfer stream: shared by all runtimes, chosen to run beside compute."""
        from .hip import transfer_stream

        return transfer_stream(device if device is not None else self.device)

    def use_stream(self, stream: Any) -> AbstractContextManager:
        from .hip import use_stream

        return use_stream(stream)

    def is_capturing(self) -> bool:
        from .hip import is_capturing

        return is_capturing()


@dataclass(frozen=True, slots=True)
class TransferTicket:
    """Readiness handle of one submitted transfer; valid until its slot is resubmitted or the runtime joins."""

    _runtime_token: object = field(repr=False)
    _event: Any = field(repr=False)
    slot: Hashable
    trace_label: str | None = None


class HipTransferRuntime:
    """Orders asynchronous transfers into ring slots against their consumers."""

    def __init__(self, device: Any = None, backend: StreamBackend | None = None) -> None:
        self.backend: StreamBackend = backend if backend is not None else HipBackend(device)
        self.transfer_stream = self.backend.new_stream(device)
        self._token = object()
        self._tickets: dict[Hashable, TransferTicket] = {}
        self._last_use: dict[Hashable, Any] = {}
        self._busy: set[Hashable] = set()
        self._active = False
        self._closed = False

    # the reference exposes these two maps to its tests under these names
    @property
    def _last_use_by_slot(self) -> dict[Hashable, Any]:
        return self._last_use

    @property
    def _active_ticket_by_slot(self) -> dict[Hashable, TransferTicket]:
        return self._tickets

    @property
    def is_active(self) -> bool:
        return self._active

    def _require_open(self) -> None:
        if self._closed:
            raise RuntimeError(f"{type(self).__name__} is closed")

    def begin(self) -> None:
        self._require_open()
        if self._active:
            raise RuntimeError(f"{type(self).__name__} is already active")
        self._last_use.clear()
        self._busy.clear()
        fork = self.backend.current_stream().record_event()
        self.transfer_stream.wait_event(fork)
        self._active = True

    def submit(self, slot: Hashable, transfer: Callable[[], None], *, trace_label: str | None = None) -> TransferTicket:
        self._require_open()
        if not self._active:
            raise RuntimeError("begin() must be called before submit()")
        if slot in self._busy:
            raise RuntimeError(f"{self._tickets[slot]} is still in use")
        last = self._last_use.get(slot)
        if last is not None:
            self.transfer_stream.wait_event(last)
        self._tickets.pop(slot, None)
        with self.backend.use_stream(self.transfer_stream):
            transfer()
        ticket = TransferTicket(self._token, self.transfer_stream.record_event(), slot, trace_label)
        self._tickets[slot] = ticket
        self._busy.add(slot)
        return ticket

    def wait_ready(self, ticket: TransferTicket, *, host: bool = False) -> None:
        """Order the current stream's next work after ``ticket``'s transfer.

        By default the current stream waits on the transfer's event. With
        ``host`` the calling thread blocks until the transfer has finished
        and the stream waits on nothing. A stream wait stays pending on the
        compute queue for as long as the transfer runs, and a host-to-device
        copy with such a waiter moves about 0.5% fewer bytes per second on
        the MI355X (35-40 us per 386 MiB copy); a blocked host costs the
        link nothing. Work the caller enqueues afterwards starts after the
        transfer, as after any host synchronisation. Under graph capture the
        transfer has not run yet, so the stream waits as by default.
        """
        self._require_open()
        if ticket._runtime_token is not self._token:
            raise ValueError(f"ticket belongs to a different {type(self).__name__}")
        if self._tickets.get(ticket.slot) is not ticket:
            raise ValueError(f"stale {ticket}")
        if host and not self.backend.is_capturing():
            ticket._event.synchronize()
            return
        self.backend.current_stream().wait_event(ticket._event)

    def finish_use(self, slot: Hashable) -> None:
        self._require_open()
        if not self._active:
            raise RuntimeError("begin() must be called before finish_use()")
        self._last_use[slot] = self.backend.current_stream().record_event()
        self._busy.discard(slot)

    def join(self) -> None:
        self._require_open()
        if self._active:
            try:
                done = self.transfer_stream.record_event()
                self.backend.current_stream().wait_event(done)
            except Exception as error:  # noqa: BLE001 - re-raised with the runtime's error type
                raise TransferStreamSynchronizationError(str(error)) from error
            self._active = False
        self._tickets.clear()
        self._last_use.clear()
        self._busy.clear()

    def close(self) -> None:
        if self._closed:
            return
        synchronize_transfer_stream(self.transfer_stream)
        self._tickets.clear()
        self._last_use.clear()
        self._busy.clear()
        self._active = False
        self._closed = True


# Drop-in name of the reference class.
CudaTransferRuntime = HipTransferRuntime
