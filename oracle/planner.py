"""Oracle: slot colouring and schedule operations, restated step by step.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). Plain Python over
small inputs; each function follows the cited reference lines. Inputs use
plain types: ``layers`` is a list of labels in execution order, sizes are a
list of (label, bytes) pairs, strategy maps are {label: [(tensor_id, bytes)]}
and layer tensors are {label: [tensor_id, ...]}.
"""

from __future__ import annotations


def adjacency(labels):
    """Path graph over labels in order (memory_block_planner.py:24-42)."""
    graph = {}
    for i in range(1, len(labels)):
        a, b = labels[i - 1], labels[i]
        graph.setdefault(b, set()).add(a)
        graph.setdefault(a, set()).add(b)
    return graph


def min_blocks_sequential(labels):
    """Greedy colouring in label order (memory_block_planner.py:44-76)."""
    if not labels:
        return 0
    graph = adjacency(labels)
    colour = {}
    for label in labels:
        taken = {colour[n] for n in graph.get(label, set()) if n in colour}
        c = 0
        while c in taken:
            c += 1
        colour[label] = c
    return max(colour.values()) + 1


def optimize_block_distribution(labels, num_blocks):
    """Least-filled legal slot per label, lowest id on ties (memory_block_planner.py:78-122)."""
    need = min_blocks_sequential(labels)
    if num_blocks < need:
        raise ValueError(f"Need at least {need} blocks")
    graph = adjacency(labels)
    blocks = {b: [] for b in range(num_blocks)}
    for label in labels:
        legal = []
        for b in range(num_blocks):
            if all(other not in graph.get(label, set()) for other in blocks[b]):
                legal.append(b)
        if not legal:
            raise ValueError(f"Cannot place layer {label} in any block")
        best = legal[0]
        for b in legal[1:]:
            if len(blocks[b]) < len(blocks[best]):
                best = b
        blocks[best].append(label)
    return {b: ls for b, ls in blocks.items() if ls}


def allocate_blocks(sizes, num_blocks, capacity=None):
    """Recursive first-fit with backtracking (memory_block_planner.py:124-216)."""
    if num_blocks <= 0:
        raise ValueError("Number of blocks must be positive")
    labels = [label for label, _ in sizes]
    size = dict(sizes)
    graph = adjacency(labels)
    blocks = {b: [] for b in range(num_blocks)}
    used = {b: 0 for b in range(num_blocks)}

    def place(i):
        if i >= len(labels):
            return True
        label = labels[i]
        for b in range(num_blocks):
            if capacity is not None and used[b] + size[label] > capacity:
                continue
            if any(other in graph.get(label, set()) for other in blocks[b]):
                continue
            blocks[b].append(label)
            used[b] += size[label]
            if place(i + 1):
                return True
            blocks[b].remove(label)
            used[b] -= size[label]
        return False

    if place(0):
        return blocks
    raise ValueError(f"Cannot allocate {len(labels)} layers to {num_blocks} blocks with given constraints")


def find_minimum_blocks(sizes, capacity=None):
    """Binary search over the slot count (memory_block_planner.py:218-252)."""
    if not sizes:
        return 0, {}
    lo, hi = 1, len(sizes)
    while lo < hi:
        mid = (lo + hi) // 2
        try:
            allocate_blocks(sizes, mid, capacity)
            hi = mid
        except ValueError:
            lo = mid + 1
    return lo, allocate_blocks(sizes, lo, capacity)


def block_sizes(sizes, allocation):
    """Largest label per slot (memory_block_planner.py:254-293)."""
    size = dict(sizes)
    return {b: (max(size[label] for label in ls) if ls else 0) for b, ls in allocation.items()}


def label_to_size_map(layers, strategy):
    """Bytes per transfer label in execution order, zeros dropped (strategy/utils.py:127-149)."""
    out = []
    for label in layers:
        total = sum(n for _, n in strategy.get(label, []))
        if total != 0:
            out.append((label, total))
    return out


def transfer_to_compute(layers, layer_tensors, strategy):
    """Compute label of each transfer's first tensor (strategy/utils.py:170-193)."""
    reader = {}
    for label in layers:
        for tid in layer_tensors.get(label, []):
            reader[tid] = label
    return {label: reader[ts[0][0]] for label, ts in strategy.items() if len(ts) > 0}


def prepare_block_strategy(layers, layer_tensors, strategy, blocks):
    """Slot plan of a strategy map (strategy/utils.py:217-260)."""
    sizes = label_to_size_map(layers, strategy)
    if blocks is None:
        _, allocation = find_minimum_blocks(sizes)
    else:
        allocation = optimize_block_distribution([label for label, _ in sizes], blocks)
    l2b = {label: b for b, ls in allocation.items() for label in ls}
    return {
        "label_to_size_map": dict(sizes),
        "allocation_ordered": allocation,
        "block_sizes": block_sizes(sizes, allocation),
        "label_to_block_id": l2b,
        "transfer_to_compute_map": transfer_to_compute(layers, layer_tensors, strategy),
    }


def find_transfers_for_preload(t2c, layers):
    """Transfers whose compute position precedes the transfer (strategy_operations.py:761-797)."""
    where = {label: i for i, label in enumerate(layers)}
    out = {}
    for t, c in t2c.items():
        tp, cp = where.get(t, -1), where.get(c, -1)
        if tp == -1 or cp == -1:
            continue
        if cp < tp:
            out[t] = c
    return out


def create_allocation_ordered(l2b, layers):
    """Group by slot, order by execution position, unknown labels last (strategy_operations.py:841-880)."""
    where = {label: i for i, label in enumerate(layers)}
    out = {}
    for label, b in l2b.items():
        out.setdefault(b, []).append(label)
    for b in out:
        out[b].sort(key=lambda label: where.get(label, float("inf")))
    return out


def _prev_compute(transfer, block, t2c, l2b, where):
    """strategy_operations.py:443-470."""
    marks = [where[c] for t, c in t2c.items() if l2b.get(t) == block]
    here = where[transfer]
    marks.append(here)
    marks.sort()
    k = marks.index(here)
    return marks[k - 1] if k > 0 else -1


def check_transfer_constraint(t2c, l2b, layers):
    """strategy_operations.py:473-522."""
    where = {label: i for i, label in enumerate(layers)}
    for t, c in t2c.items():
        tp = where.get(t, -1)
        if tp == -1 or l2b.get(t) is None:
            continue
        prev = _prev_compute(t, l2b[t], t2c, l2b, where)
        if prev != -1 and tp < prev:
            return False
    return True


def check_overlap_constraint(t2c, layers, l2b):
    """strategy_operations.py:525-620."""
    where = {label: i for i, label in enumerate(layers)}
    n = len(layers)
    per_block = {}
    for t, c in t2c.items():
        b = l2b.get(t)
        if b is None:
            continue
        per_block.setdefault(b, []).append((t, c))
    for pairs in per_block.values():
        spans = []
        for t, c in pairs:
            tp, cp = where.get(t, -1), where.get(c, -1)
            if tp == -1 or cp == -1:
                continue
            spans.append((tp, cp))
        kinds = {}
        for tp, cp in spans:
            kinds.setdefault(tp, set()).add("transfer")
            kinds.setdefault(cp, set()).add("compute")
        if any(k == {"transfer", "compute"} for k in kinds.values()):
            return False
        for i in range(len(spans)):
            for j in range(len(spans)):
                if i >= j:
                    continue
                t1, c1 = spans[i]
                t2, c2 = spans[j]
                r1 = (set(range(t1, n)) | set(range(c1 + 1))) if c1 < t1 else set(range(t1, c1 + 1))
                r2 = (set(range(t2, n)) | set(range(c2 + 1))) if c2 < t2 else set(range(t2, c2 + 1))
                if r1 & r2:
                    return False
    return True


def rearrange_transfers(t2c, l2b, layers, gap=1):
    """Move transfers to the earliest legal free position (strategy_operations.py:623-758)."""
    if not t2c or not l2b or not layers:
        return dict(t2c), dict(l2b), {}
    where = {label: i for i, label in enumerate(layers)}
    name = {i: label for i, label in enumerate(layers)}
    n = len(layers)
    new_t2c, new_l2b, remapped = dict(t2c), dict(l2b), {}
    order = [(t, c, l2b[t]) for t, c in t2c.items() if l2b.get(t) is not None]
    for t, c, b in order:
        taken = {where[x] for x in new_t2c if x in where}
        free = set(range(n)) - taken
        prev = _prev_compute(t, b, new_t2c, new_l2b, where)
        tp, cp = where[t], where[c]
        if prev == -1:
            slots = free & set(range(cp))
        else:
            lo = prev + gap
            if cp < lo:
                slots = free & (set(range(cp)) | set(range(lo, n)))
            else:
                slots = free & set(range(lo, cp))
        slots.add(tp)
        best_gap, best = -1, -1
        for s in slots:
            g = cp - s if s < cp else n - s + cp
            if g > best_gap:
                best_gap, best = g, s
        target = name.get(best)
        if target is not None:
            del new_t2c[t]
            del new_l2b[t]
            new_t2c[target] = c
            new_l2b[target] = b
            remapped[t] = target
    if not check_transfer_constraint(new_t2c, new_l2b, layers):
        raise ValueError("Transfer constraint violated after optimization.")
    if not check_overlap_constraint(new_t2c, layers, new_l2b):
        raise ValueError("Overlap constraint violated after optimization.")
    return new_t2c, new_l2b, remapped
