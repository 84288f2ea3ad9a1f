"""Oracle: stream/event operation traces of the pipelined loaders.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). Replays a sequence
of ``enter`` / ``forward`` / ``exit`` calls through a restatement of the
reference's transfer runtime (core/transfer.py:39-146) and both block loaders
(loaders.py:1473-1658 default, loaders.py:1661-1858 reordered) and returns
the operations they issue, as ``(op, stream, target)`` tuples:

* ``("record_event", stream, event_name)``
* ``("wait_event", stream, event_name)``
* ``("schedule_transfer", "transfer", label)``
* ``("forward", "compute", label)``
* ``("wait_stream", stream, other_stream)``

Event names are ``<stream>_ev_<n>`` with one counter across both streams,
counted from the first call after construction (the reference test resets its
counter after building the loader, test_loader_synchronization.py:204-206).
"""

from __future__ import annotations


class _Sim:
    def __init__(self):
        self.log = []
        self.count = 0

    def record(self, stream):
        self.count += 1
        name = f"{stream}_ev_{self.count}"
        self.log.append(("record_event", stream, name))
        return name

    def wait(self, stream, event):
        self.log.append(("wait_event", stream, event))


class _Runtime:
    """core/transfer.py:39-146 with streams 'compute' and 'transfer'."""

    def __init__(self, sim):
        self.sim = sim
        self.tickets = {}      # slot -> ticket id
        self.last_use = {}     # slot -> event
        self.busy = set()
        self.active = False
        self.next_ticket = 0

    def begin(self):
        if self.active:
            raise RuntimeError("already active")
        self.last_use.clear()
        self.busy.clear()
        ev = self.sim.record("compute")
        self.sim.wait("transfer", ev)
        self.active = True

    def submit(self, slot, label):
        if not self.active:
            raise RuntimeError("begin() must be called before submit()")
        if slot in self.busy:
            raise RuntimeError("still in use")
        if slot in self.last_use:
            self.sim.wait("transfer", self.last_use[slot])
        self.tickets.pop(slot, None)
        self.sim.log.append(("schedule_transfer", "transfer", label))
        ev = self.sim.record("transfer")
        self.next_ticket += 1
        ticket = (self.next_ticket, slot, ev)
        self.tickets[slot] = ticket
        self.busy.add(slot)
        return ticket

    def wait_ready(self, ticket):
        if self.tickets.get(ticket[1]) is not ticket:
            raise ValueError("stale ticket")
        self.sim.wait("compute", ticket[2])

    def finish_use(self, slot):
        if not self.active:
            raise RuntimeError("begin() must be called before finish_use()")
        self.last_use[slot] = self.sim.record("compute")
        self.busy.discard(slot)

    def join(self):
        if self.active:
            ev = self.sim.record("transfer")
            self.sim.wait("compute", ev)
            self.active = False
        self.tickets.clear()
        self.last_use.clear()
        self.busy.clear()


def _preload_set(t2c, layers):
    where = {label: i for i, label in enumerate(layers)}
    return {t: c for t, c in t2c.items() if t in where and c in where and where[c] < where[t]}


def trace(kind, layers, t2c, l2b, calls, *, reload_after_abort=False):
    """Operations issued for ``calls`` (a list of ('enter'|'forward'|'exit'|'join', label)).

    ``kind`` is ``"default"`` or ``"reordered"``. Construction (with its
    preload) is not part of the returned trace.

    ``reload_after_abort`` models one deliberate difference of the product
    from the reference: after the abort recovery at the first label (a pass
    that never reached its last label), the cyclic preload transfers are
    issued again, because the aborted pass never issued the transfers that
    fill the next pass's first slots. The reference (loaders.py:1729-1740)
    only joins and clears; its default is kept here.
    """
    sim = _Sim()
    rt = _Runtime(sim)
    consumes = {}
    for t, c in t2c.items():
        consumes.setdefault(c, []).append(l2b[t])
    first = layers[0] if layers else None
    last = layers[-1] if layers else None
    scheduled = {}
    preloaded_consumers = set()
    pre = _preload_set(t2c, layers)
    if pre:
        rt.begin()
        for t, c in pre.items():
            rt.submit(l2b[t], t)
            preloaded_consumers.add(c)
        rt.join()
    sim.log.clear()
    sim.count = 0

    def release(label):
        slots = consumes.get(label)
        if rt.active and slots:
            for s in slots:
                rt.finish_use(s)
        else:
            sim.record("compute")

    def end_if_last(label):
        if label == last:
            if rt.active:
                rt.join()
            scheduled.clear()

    for op, label in calls:
        if op == "forward":
            sim.log.append(("forward", "compute", label))
        elif op == "join":
            rt.join()
            scheduled.clear()
        elif op == "enter":
            if label == first and rt.active:
                rt.join()
                scheduled.clear()
                if reload_after_abort and pre:
                    rt.begin()
                    for t in pre:
                        rt.submit(l2b[t], t)
                    rt.join()
            if not rt.active:
                rt.begin()
            if kind == "reordered":
                for ticket in scheduled.pop(label, []):
                    rt.wait_ready(ticket)
                if label in l2b:
                    scheduled.setdefault(t2c[label], []).append(rt.submit(l2b[label], label))
            else:
                if label in l2b:
                    scheduled[label] = rt.submit(l2b[label], label)
        elif op == "exit":
            if kind == "default" and label in scheduled:
                rt.wait_ready(scheduled[label])
            release(label)
            end_if_last(label)
        else:
            raise ValueError(op)
    return sim.log


def passes(labels, n=1):
    """The call sequence of ``n`` full passes over ``labels``."""
    out = []
    for _ in range(n):
        for label in labels:
            out += [("enter", label), ("forward", label), ("exit", label)]
    return out
