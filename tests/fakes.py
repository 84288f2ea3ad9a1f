"""Recording stand-ins for streams, events and controllers (no GPU needed).

Mirrors the recorder the reference uses for its ordering tests
(tests/unit/test_loader_synchronization.py:37-137): every stream operation is
appended to one log; events carry a ``completed`` flag so a wait on an
unfinished event is marked as a stall.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field


@dataclass
class FakeEvent:
    name: str
    completed: bool = True
    rec: "Recorder | None" = field(default=None, repr=False, compare=False)

    def synchronize(self) -> None:
        """A host wait: logged on the "host" stream, stalled when the event had not completed."""
        if self.rec is not None:
            self.rec.log.append(Entry("synchronize_event", "host", self.name, not self.completed))
        self.completed = True


@dataclass
class Entry:
    op: str
    stream: str
    target: str
    stalled: bool = False


@dataclass
class Recorder:
    log: list[Entry] = field(default_factory=list)
    counter: int = 0

    def new_event(self, stream: str, completed: bool) -> FakeEvent:
        self.counter += 1
        return FakeEvent(f"{stream}_ev_{self.counter}", completed, self)

    def forward(self, label: str) -> None:
        self.log.append(Entry("forward", "compute", label))

    def ops(self) -> list[tuple[str, str]]:
        return [(e.op, e.stream) for e in self.log]

    def triples(self) -> list[tuple[str, str, str]]:
        return [(e.op, e.stream, e.target) for e in self.log]

    def find(self, op: str, target: str | None = None, stream: str | None = None) -> list[int]:
        return [i for i, e in enumerate(self.log)
                if e.op == op and (target is None or e.target == target) and (stream is None or e.stream == stream)]

    def dump(self) -> str:
        return "\n".join(f"[{i:3d}] {e}" for i, e in enumerate(self.log))


class FakeStream:
    def __init__(self, name: str, rec: Recorder, completes: bool = True) -> None:
        self.name = name
        self.rec = rec
        self.completes = completes
        self.fail_on: set[str] = set()

    def record_event(self, event=None):
        if "record_event" in self.fail_on:
            raise RuntimeError("record_event failed")
        ev = self.rec.new_event(self.name, self.completes)
        self.rec.log.append(Entry("record_event", self.name, ev.name))
        return ev

    def wait_event(self, ev: FakeEvent) -> None:
        if "wait_event" in self.fail_on:
            raise RuntimeError("wait_event failed")
        self.rec.log.append(Entry("wait_event", self.name, ev.name, not ev.completed))
        ev.completed = True

    def wait_stream(self, other: "FakeStream") -> None:
        self.rec.log.append(Entry("wait_stream", self.name, other.name))

    def synchronize(self) -> None:
        if "synchronize" in self.fail_on:
            raise RuntimeError("synchronize failed")
        self.rec.log.append(Entry("synchronize", self.name, ""))


class FakeBackend:
    """compute = torch's current stream; transfer = the stream the runtime creates."""

    def __init__(self, rec: Recorder, slow_transfer: bool = False) -> None:
        self.rec = rec
        self.compute = FakeStream("compute", rec)
        self.transfer = FakeStream("transfer", rec, completes=not slow_transfer)
        self.current = self.compute
        self.created = 0
        self.capturing = False

    def current_stream(self):
        return self.current

    def new_stream(self, device):
        self.created += 1
        return self.transfer

    @contextmanager
    def use_stream(self, stream):
        prev, self.current = self.current, stream
        try:
            yield
        finally:
            self.current = prev

    def is_capturing(self) -> bool:
        return self.capturing


class FakeController:
    """Records ``schedule_transfer`` and the stream that was current when it ran."""

    def __init__(self, rec: Recorder, backend: FakeBackend | None = None) -> None:
        self.rec = rec
        self.backend = backend
        self.streams_seen: list[str] = []

    def schedule_transfer(self, label: str, non_blocking: bool = True) -> None:
        if self.backend is not None:
            self.streams_seen.append(self.backend.current_stream().name)
        self.rec.log.append(Entry("schedule_transfer", "transfer", label))

    def get_gpu_memory_bytes(self) -> int:
        return 0

    def shutdown(self) -> None:
        return None
