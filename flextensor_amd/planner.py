"""Ring-slot planning and transfer-schedule surgery (row a9 of the hot path).

Labels are offload units in execution order. Two labels that run back to back
must not share a GPU slot, so the slot assignment is a colouring of the path
graph of labels (memory_block_planner.py:12-294); a slot is sized to its
largest label. The schedule maps each transfer label to the compute label
that consumes its bytes (strategy/utils.py:170-193); transfers whose consumer
runs earlier in the pass are issued before the first pass (cyclic preload,
strategy_operations.py:761-797), and transfers can be moved earlier into
labels that issue no transfer of their own (strategy_operations.py:623-758).

The result handed to loaders is :class:`BlockStrategyData`
(strategy/protocol.py:36-57).
"""

from __future__ import annotations

from collections import OrderedDict
from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field


@dataclass(frozen=True)
class TensorStatistics:
    """One managed tensor: its id, name, size and measured load time (collectors.py:11-19)."""

    tensor_id: int
    name: str
    size_bytes: int
    load_time_ms: float = 0.0


@dataclass(frozen=True)
class LayerStatistics:
    """One offload unit in execution order with the tensors it reads (collectors.py:22-30)."""

    label: str
    tensors: list[TensorStatistics] = field(default_factory=list)
    duration: float = 0.0


@dataclass
class BlockStrategyData:
    """Everything a block loader needs to run the pipelined transfers."""

    label_to_size_map: dict[str, int]
    allocation_ordered: dict[int, list[str]]
    block_sizes: dict[int, int]
    label_to_block_id: dict[str, int]
    transfer_to_compute_map: dict[str, str]


class MemoryBlockPlanner:
    """Assigns labels to ring slots so that neighbouring labels never share one."""

    def __init__(self, layer_sizes: Mapping[str, int]) -> None:
        self.layer_sizes = OrderedDict(layer_sizes)
        self.layers = list(self.layer_sizes)
        self._index = {label: i for i, label in enumerate(self.layers)}
        self.adjacency_graph = self._path_graph()

    def _path_graph(self) -> dict[str, set[str]]:
        g: dict[str, set[str]] = {}
        for a, b in zip(self.layers, self.layers[1:]):
            g.setdefault(a, set()).add(b)
            g.setdefault(b, set()).add(a)
        return g

    def _neighbours(self, label: str) -> set[str]:
        return self.adjacency_graph.get(label, set())

    def find_minimum_blocks_sequential(self) -> int:
        """Chromatic number of the label path: 0, 1, or 2 for two or more labels."""
        return min(len(self.layers), 2)

    def optimize_block_distribution(self, num_blocks: int) -> dict[int, list[str]]:
        """Place labels in order, each into the least-filled slot that holds no neighbour.

        Ties go to the lowest slot id; empty slots are dropped from the result.
        """
        need = self.find_minimum_blocks_sequential()
        if num_blocks < need:
            raise ValueError(f"Need at least {need} blocks")
        members: list[list[str]] = [[] for _ in range(num_blocks)]
        slot_of: dict[str, int] = {}
        for label in self.layers:
            banned = {slot_of[n] for n in self._neighbours(label) if n in slot_of}
            choices = [b for b in range(num_blocks) if b not in banned]
            if not choices:
                raise ValueError(f"Cannot place layer {label} in any block")
            best = min(choices, key=lambda b: (len(members[b]), b))
            members[best].append(label)
            slot_of[label] = best
        return {b: labels for b, labels in enumerate(members) if labels}

    def allocate_blocks(self, num_blocks: int, block_capacity: int | None = None) -> dict[int, list[str]]:
        """First-fit placement with backtracking under an optional per-slot byte capacity."""
        if num_blocks <= 0:
            raise ValueError("Number of blocks must be positive")
        members: list[list[str]] = [[] for _ in range(num_blocks)]
        used = [0] * num_blocks

        # Iterative depth-first search over (label index, next slot to try).
        choice = [0] * len(self.layers)
        i = 0
        while 0 <= i < len(self.layers):
            label = self.layers[i]
            size = self.layer_sizes[label]
            placed = False
            for b in range(choice[i], num_blocks):
                fits = block_capacity is None or used[b] + size <= block_capacity
                if fits and not (self._neighbours(label) & set(members[b])):
                    members[b].append(label)
                    used[b] += size
                    choice[i] = b
                    placed = True
                    break
            if placed:
                i += 1
                if i < len(self.layers):
                    choice[i] = 0
                continue
            # undo the previous label and try its next slot
            choice[i] = 0
            i -= 1
            if i >= 0:
                prev = self.layers[i]
                members[choice[i]].remove(prev)
                used[choice[i]] -= self.layer_sizes[prev]
                choice[i] += 1
        if i < 0:
            raise ValueError(
                f"Cannot allocate {len(self.layers)} layers to {num_blocks} blocks with given constraints"
            )
        return {b: labels for b, labels in enumerate(members)}

    def find_minimum_blocks(self, block_capacity: int | None = None) -> tuple[int, dict[int, list[str]]]:
        """Smallest slot count for which :meth:`allocate_blocks` succeeds (binary search)."""
        if not self.layers:
            return 0, {}
        lo, hi = 1, len(self.layers)
        while lo < hi:
            mid = (lo + hi) // 2
            try:
                self.allocate_blocks(mid, block_capacity)
                hi = mid
            except ValueError:
                lo = mid + 1
        return lo, self.allocate_blocks(lo, block_capacity)

    def find_minimum_block_sizes(self, allocation: Mapping[int, Sequence[str]]) -> dict[int, int]:
        """Bytes of each slot: the largest label assigned to it (0 for an empty slot)."""
        return {b: max((self.layer_sizes[label] for label in labels), default=0) for b, labels in allocation.items()}


# ---------------------------------------------------------------------------
# block-strategy glue (strategy/utils.py:127-290)
# ---------------------------------------------------------------------------


def compute_label_to_size_map(
    layer_stats: Sequence[LayerStatistics], strategy_map: Mapping[str, Sequence[TensorStatistics]]
) -> OrderedDict[str, int]:
    """Bytes transferred at each label, in execution order, zero-byte labels dropped."""
    out: OrderedDict[str, int] = OrderedDict()
    for layer in layer_stats:
        n = sum(t.size_bytes for t in strategy_map.get(layer.label, ()))
        if n:
            out[layer.label] = n
    return out


def calculate_transfer_to_compute_map(
    layer_stats: Sequence[LayerStatistics], strategy_map: Mapping[str, Sequence[TensorStatistics]]
) -> dict[str, str]:
    """Transfer label -> label that computes with the first tensor it transfers (last reader wins)."""
    reader: dict[int, str] = {}
    for layer in layer_stats:
        for t in layer.tensors:
            reader[t.tensor_id] = layer.label
    return {label: reader[ts[0].tensor_id] for label, ts in strategy_map.items() if ts}


def reverse_transfer_to_compute_map(t2c: Mapping[str, str]) -> dict[str, str]:
    out: dict[str, str] = {}
    for transfer, compute in t2c.items():
        if compute in out:
            raise ValueError(f"Compute label '{compute}' mapped from both '{out[compute]}' and '{transfer}'")
        out[compute] = transfer
    return out


def label_to_block_id_from(allocation: Mapping[int, Sequence[str]]) -> dict[str, int]:
    return {label: b for b, labels in allocation.items() for label in labels}


def prepare_block_strategy(
    strategy_map: Mapping[str, Sequence[TensorStatistics]],
    layer_stats: Sequence[LayerStatistics],
    blocks: int | None,
) -> BlockStrategyData:
    """Slot plan for a strategy map: ``blocks`` slots, or the minimum when ``None``."""
    sizes = compute_label_to_size_map(layer_stats, strategy_map)
    planner = MemoryBlockPlanner(sizes)
    if blocks is None:
        _, allocation = planner.find_minimum_blocks()
    else:
        allocation = planner.optimize_block_distribution(blocks)
    return BlockStrategyData(
        label_to_size_map=dict(sizes),
        allocation_ordered=allocation,
        block_sizes=planner.find_minimum_block_sizes(allocation),
        label_to_block_id=label_to_block_id_from(allocation),
        transfer_to_compute_map=calculate_transfer_to_compute_map(layer_stats, strategy_map),
    )


# ---------------------------------------------------------------------------
# schedule surgery (strategy_operations.py:389-880)
# ---------------------------------------------------------------------------


def positions(layer_stats: Sequence[LayerStatistics]) -> dict[str, int]:
    return {layer.label: i for i, layer in enumerate(layer_stats)}


def find_transfers_for_preload(t2c: Mapping[str, str], layer_stats: Sequence[LayerStatistics]) -> dict[str, str]:
    """Transfers whose consumer runs earlier in the pass than the transfer itself.

    These wrap around the pass boundary and must be issued before the first pass.
    """
    pos = positions(layer_stats)
    return {t: c for t, c in t2c.items() if t in pos and c in pos and pos[c] < pos[t]}


def create_allocation_ordered(
    label_to_block_id: Mapping[str, int], layer_stats: Sequence[LayerStatistics]
) -> dict[int, list[str]]:
    """Slot id -> its labels in execution order (labels not in the pass go last, in input order)."""
    pos = positions(layer_stats)
    groups: dict[int, list[str]] = {}
    for label, b in label_to_block_id.items():
        groups.setdefault(b, []).append(label)
    end = len(pos)
    return {b: sorted(labels, key=lambda x: pos.get(x, end)) for b, labels in groups.items()}


def remap_strategy(strategy_map: Mapping[str, Sequence] | None, key_remap: Mapping[str, str]) -> dict[str, Sequence]:
    """Rename strategy-map keys; keys without a new name stay."""
    if not strategy_map:
        return {} if strategy_map is None else dict(strategy_map)
    out = dict(strategy_map)
    for old, new in key_remap.items():
        if old in strategy_map:
            out[new] = strategy_map[old]
            if old != new:
                del out[old]
    return out


def _cyclic_range(start: int, end: int, n: int) -> set[int]:
    """Positions visited going from ``start`` to ``end`` inclusive, wrapping at ``n``."""
    if end < start:
        return set(range(start, n)) | set(range(end + 1))
    return set(range(start, end + 1))


def _previous_compute_position(transfer: str, block: int, t2c: Mapping[str, str],
                               l2b: Mapping[str, int], pos: Mapping[str, int]) -> int:
    """Position of the compute that last used ``block`` before ``transfer`` runs (-1: none)."""
    here = pos[transfer]
    marks = sorted([pos[c] for t, c in t2c.items() if l2b.get(t) == block] + [here])
    i = marks.index(here)
    return marks[i - 1] if i > 0 else -1


def check_transfer_constraint(t2c: Mapping[str, str], l2b: Mapping[str, int],
                              layer_stats: Sequence[LayerStatistics]) -> bool:
    """No transfer runs before the previous consumer of its slot."""
    pos = positions(layer_stats)
    for transfer in t2c:
        if transfer not in pos:
            continue
        block = l2b.get(transfer)
        if block is None:
            continue
        prev = _previous_compute_position(transfer, block, t2c, l2b, pos)
        if prev != -1 and pos[transfer] < prev:
            return False
    return True


def check_overlap_constraint(t2c: Mapping[str, str], layer_stats: Sequence[LayerStatistics],
                             l2b: Mapping[str, int]) -> bool:
    """Within one slot, no transfer shares a position with a compute and no two
    transfer->compute windows (cyclic) overlap."""
    pos = positions(layer_stats)
    n = len(layer_stats)
    by_block: dict[int, list[tuple[int, int]]] = {}
    for t, c in t2c.items():
        b = l2b.get(t)
        if b is None or t not in pos or c not in pos:
            continue
        by_block.setdefault(b, []).append((pos[t], pos[c]))
    for pairs in by_block.values():
        transfers = {tp for tp, _ in pairs}
        computes = {cp for _, cp in pairs}
        if transfers & computes:
            return False
        windows = [_cyclic_range(tp, cp, n) for tp, cp in pairs]
        for i in range(len(windows)):
            for j in range(i + 1, len(windows)):
                if windows[i] & windows[j]:
                    return False
    return True


def rearrange_transfers(
    transfer_to_compute_map: Mapping[str, str],
    label_to_block_id: Mapping[str, int],
    layer_stats: Sequence[LayerStatistics],
    min_compute_transfer_gap: int = 1,
) -> tuple[dict[str, str], dict[str, int], dict[str, str]]:
    """Move each transfer to the free label furthest ahead of its consumer.

    A label is free when no transfer is issued there. The move is bounded by
    the previous consumer of the same slot (plus ``min_compute_transfer_gap``),
    so a slot is never overwritten while still in use. Moves are applied in
    the input order of the map; moved entries are re-inserted at the end.
    Returns ``(t2c, label_to_block_id, remapped)`` where ``remapped`` maps each
    moved transfer label to its new label.
    """
    if not transfer_to_compute_map or not label_to_block_id or not layer_stats:
        return dict(transfer_to_compute_map), dict(label_to_block_id), {}
    pos = positions(layer_stats)
    at = {i: layer.label for i, layer in enumerate(layer_stats)}
    n = len(layer_stats)
    t2c = dict(transfer_to_compute_map)
    l2b = dict(label_to_block_id)
    remapped: dict[str, str] = {}
    order = [(t, c, label_to_block_id[t]) for t, c in transfer_to_compute_map.items() if t in label_to_block_id]
    for transfer, compute, block in order:
        occupied = {pos[t] for t in t2c if t in pos}
        free = set(range(n)) - occupied
        prev = _previous_compute_position(transfer, block, t2c, l2b, pos)
        c_pos = pos[compute]
        if prev == -1:
            window = set(range(c_pos))
        else:
            lo = prev + min_compute_transfer_gap
            window = set(range(lo, c_pos)) if c_pos >= lo else set(range(c_pos)) | set(range(lo, n))
        candidates = (free & window) | {pos[transfer]}
        # lead time of issuing at position p for a consumer at c_pos (cyclic)
        best = max(candidates, key=lambda p: c_pos - p if p < c_pos else n - p + c_pos)
        new_label = at[best]
        del t2c[transfer]
        del l2b[transfer]
        t2c[new_label] = compute
        l2b[new_label] = block
        remapped[transfer] = new_label
    if not check_transfer_constraint(t2c, l2b, layer_stats):
        raise ValueError("Transfer constraint violated after optimization.")
    if not check_overlap_constraint(t2c, layer_stats, l2b):
        raise ValueError("Overlap constraint violated after optimization.")
    return t2c, l2b, remapped
