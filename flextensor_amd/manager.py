"""``offload(model, config)``: the reference's entry point and phase contract.

Phases advance after each forward of the root module, as in the reference
(offload_manager.py:297-303, 1747-1820): ``DISCOVERY`` (execution order of
the offload units), ``PROFILING`` (per-unit compute time), then
``INFERENCE``, when the plan is computed and the streaming loader is built
(offload_manager.py:1714-1728; tensor_manager.py:1661-1800):

1. unit tensors are packed per transfer label into pinned blocks and the
   streamed parameters alias typed views of GPU ring slots
   (tensor_processors.py:802-833);
2. units kept resident and every tensor outside the units are placed on the
   GPU by stream-and-scatter (the role of tensor_processors.py:685-742);
3. each unit's forward is wrapped in a trap that calls ``loader.enter`` /
   ``loader.exit`` (trap_tensor_mode.py:376-397).

During discovery and profiling a unit's tensors are loaded synchronously on
``enter`` and dropped on ``exit`` (the role of the warm-up and profile
loaders).

Units are modules chosen by ``include_patterns`` (their forwards are
patched) or, when no module is chosen, manual ``offload_block(label)``
regions of the caller's code (offload_manager.py:2251-2298). A manual
block's tensors are found during discovery by watching which parameters the
code inside the block hands to torch functions (the role of the reference's
trap tensor mode, trap_tensor_mode.py): the model's parameters stay on the
host until first used; one used inside a single block belongs to it and is
uploaded for the block's duration, one used outside blocks or by two blocks
is placed on the GPU for good. The plan keeps every unit resident when the budget allows, and
otherwise streams the fewest units that fit the budget, spread evenly over
the pass; slots are added while the slot-reuse check of the reference
(strategy_operations.py:525-620) reports a hazard.
"""

from __future__ import annotations

import contextlib
import dataclasses
import logging
import os
import threading
import time
import types
from collections.abc import Callable, Iterator, Mapping, Sequence
from dataclasses import dataclass, field
from enum import Enum
from typing import Any

import torch
from torch import nn
from torch.overrides import TorchFunctionMode
from torch.utils._pytree import tree_leaves

from . import _native as nat
from . import custom_ops, hip
from .allocation_block import HostPinner
from .config import OffloadConfig
from .controllers import AllocationBlockController, RawBlockController
from .layout import overlapping_views
from .link_model import (LinkMeasurement, MemoryTransferInterpolator, encoding_pays, format_memory_transfer_table,
                         is_link_bound, link_probe_sizes, measure_link)
from .loaders import PreallocatedBatchTransferTensorLoader, PreallocatedBatchTransferTensorLoaderReordered
from .planner import (
    BlockStrategyData,
    LayerStatistics,
    TensorStatistics,
    check_overlap_constraint,
    create_allocation_ordered,
    prepare_block_strategy,
    rearrange_transfers,
    remap_strategy,
)
from .prefetch_policy import PiecewisePrefetchPolicy
from .profile import TensorManagerState, load_state, save_state
from .replan import (REPLAN_MEASURE_PASSES, REPLAN_WARMUP_PASSES, StrategyReplanState, StrategyReplanStatus,
                     measured_compute, replanned_link)
from .scatter import upload_tensors
from .selection import parameter_filter, select_offload_units
from .timing import OffloadTimingCollector, OffloadTimingReport
from .transfer import TransferStreamSynchronizationError

LOGGER = logging.getLogger(__name__)
DEFAULT_MANAGER_NAME = "default"
MIN_GPU_BUDGET_BYTES = 256 * 1024**2  # below this much available memory a budget cannot be met


class OffloadPhase(Enum):
    NOT_INITIALIZED = "not_initialized"
    DISCOVERY = "discovery"
    PROFILING = "profiling"
    INFERENCE = "inference"


@dataclass
class GPUMemoryUsage:
    """GPU bytes held by ring slots and by tensors placed permanently (types.py:13-59).

    ``total_bytes`` defaults to the sum of the two parts.
    """

    blocks_bytes: int = 0
    unmapped_tensors_bytes: int = 0
    total_bytes: int | None = None

    def __post_init__(self) -> None:
        if self.total_bytes is None:
            self.total_bytes = self.blocks_bytes + self.unmapped_tensors_bytes

    @property
    def blocks_mb(self) -> float:
        return self.blocks_bytes / (1024 * 1024)

    @property
    def unmapped_tensors_mb(self) -> float:
        return self.unmapped_tensors_bytes / (1024 * 1024)

    @property
    def total_mb(self) -> float:
        return self.total_bytes / (1024 * 1024)


@dataclass
class StreamPlan:
    """What the planner decided: streamed and resident units plus the slot plan."""

    streamed: list[str]
    resident: list[str]
    block_data: BlockStrategyData | None
    strategy_map: dict[str, list[TensorStatistics]]
    reordered: bool
    budget_bytes: int | None
    planned_gpu_bytes: int
    # resident units kept encoded in HBM (encode_resident_blocks), and the device bytes each reserves
    encoded_resident: dict[str, int] = field(default_factory=dict)


class _CompiledCall(threading.local):
    active = False


_COMPILED_CALL = _CompiledCall()


def raise_dynamo_limits(n_units: int) -> None:
    """Raise the compiler's recompile limits so each of ``n_units`` units keeps its own graph.

    Each unit's forward closes over its own label, so the compiler specializes
    once per unit; with more units than the default limit (8) the rest would
    silently run uncompiled. Limits are only raised (compiled_offload.py:24-46).
    """
    if n_units <= 0:
        return
    import torch._dynamo as dynamo

    needed = 2 * n_units + 16
    for attr in ("recompile_limit", "cache_size_limit", "accumulated_recompile_limit",
                 "accumulated_cache_size_limit"):
        if hasattr(dynamo.config, attr) and (getattr(dynamo.config, attr) or 0) < needed:
            setattr(dynamo.config, attr, needed)


@dataclass
class _Unit:
    label: str
    module: nn.Module | None  # None for a manual ``offload_block`` region
    params: list[nn.Parameter] = field(default_factory=list)
    names: list[str] = field(default_factory=list)  # qualified parameter names, parallel to params
    compiled: Callable[..., Any] | None = None  # compile_fn(module), installed at INFERENCE

    @property
    def nbytes(self) -> int:
        return sum(p.numel() * p.element_size() for p in self.params)

    def stats(self, duration: float = 0.0) -> LayerStatistics:
        names = self.names or [f"{self.label}.{i}" for i in range(len(self.params))]
        return LayerStatistics(self.label, [TensorStatistics(id(p), n, p.numel() * p.element_size())
                                            for p, n in zip(self.params, names)], duration)


def encode_residents(resident: Sequence[str], raw_bytes: Mapping[str, int],
                     encodable: Mapping[str, tuple[int, int]], room: int) -> tuple[dict[str, int], int] | None:
    """The fewest resident units to keep encoded in HBM so that the residents fit ``room`` bytes.

    ``encodable[label]`` is (device bytes reserved for its encoded block, bytes of its packed raw block).
    The units kept encoded share one decode slot, as large as the largest of their packed raw blocks,
    counted once. Units are taken by the bytes they save, largest first (ties: earlier in the pass).
    Returns ({label: reserved bytes}, resident bytes including the decode slot), or None when even
    encoding every candidate does not fit."""
    placed = sum(raw_bytes[x] for x in resident)
    if placed <= room:
        return {}, placed
    pos = {x: i for i, x in enumerate(resident)}
    cands = sorted((x for x in resident if x in encodable and encodable[x][0] < raw_bytes[x]),
                   key=lambda x: (encodable[x][0] - raw_bytes[x], pos[x]))
    chosen: dict[str, int] = {}
    slot = 0
    for x in cands:
        placed -= raw_bytes[x] - encodable[x][0]
        slot = max(slot, encodable[x][1])
        chosen[x] = encodable[x][0]
        if placed + slot <= room:
            return chosen, placed + slot
    return None


def plan_streaming(units: Sequence[_Unit], order: Sequence[str], budget: int | None, base_bytes: int,
                   num_blocks: int, min_blocks: int | None = None,
                   encodable: Mapping[str, tuple[int, int]] | None = None) -> StreamPlan:
    """Choose streamed units and the slot plan under a GPU byte budget.

    The fewest units stream that fit, spread evenly over the pass: the
    picks centred in k equal spans, rotated so the first unit streams (the
    gaps between consecutive picks, the last to the first included, are the
    centred ones). A streamed first unit is loaded by a cyclic transfer
    issued at the previous pass's last units, so the ring keeps the link busy
    across the pass boundary; a first transfer issued inside the pass would
    wait for the fork at the pass start, behind the previous pass's tail
    compute. For that choice the slot count is the largest in
    ``[min_blocks, num_blocks]`` whose
    slots fit the budget (the deepest prefetch the memory allows; the
    reference searches the same range, config.py:207-225). Slots beyond
    ``num_blocks`` are added only while the reference's slot-reuse check
    reports a hazard.

    With ``encodable`` (``encode_resident_blocks``: per unit, the device
    bytes of its encoded block and the bytes of its packed raw block) a
    resident set that does not fit raw may keep some units encoded in HBM
    (:func:`encode_residents`), so fewer units stream for the same budget.
    Such a plan is chosen for the fewest streamed bytes, not the fewest
    streamed units: of unequal units the fewest may not be the smallest
    (counts up to twice the first that fits are compared).
    """
    by_label = {u.label: u for u in units}
    labels = list(order)
    sizes = [by_label[x].nbytes for x in labels]
    total = base_bytes + sum(sizes)
    if budget is not None and total <= budget:
        return StreamPlan([], labels, None, {}, False, budget, total)
    n = len(labels)
    stats = [by_label[x].stats() for x in labels]
    hi = max(num_blocks, 2)
    lo = max(2, min(hi, min_blocks if min_blocks is not None else hi))
    def attempt(k: int) -> StreamPlan | None:
        centred = sorted({min(n - 1, int((i + 0.5) * n / k)) for i in range(k)})
        pick = [i - centred[0] for i in centred]
        if len(pick) < k:
            return None
        streamed = [labels[i] for i in pick]
        if budget is None and k < n:
            return None
        # i == 0 wraps to the last label: a cyclic preload
        strategy = {labels[i - 1]: list(stats[i].tensors) for i in pick}
        resident = [x for x in labels if x not in streamed]
        placed = base_bytes + sum(by_label[x].nbytes for x in resident)
        chosen = None
        hazard_free = False
        for blocks in [*range(hi, lo - 1, -1), *range(hi + 1, n + 3)]:
            bd = prepare_block_strategy(strategy, stats, blocks)
            if not check_overlap_constraint(bd.transfer_to_compute_map, stats, bd.label_to_block_id):
                continue
            hazard_free = True
            ring = sum(bd.block_sizes.values())
            gpu = placed + ring
            enc: dict[str, int] = {}
            if budget is not None and encodable and gpu > budget:
                got = encode_residents(resident, {x: by_label[x].nbytes for x in resident}, encodable,
                                       budget - base_bytes - ring)
                if got is not None:
                    enc, gpu = got[0], base_bytes + got[1] + ring
            if budget is None or gpu <= budget:
                chosen = (bd, gpu, enc)
                break
            if blocks > hi:
                break  # extra slots only grow the footprint
        if not hazard_free:
            raise RuntimeError("no hazard-free slot plan found")
        if chosen is None:
            return None
        bd, gpu, enc = chosen
        reordered = bool(resident)
        if reordered:
            t2c, l2b, remapped = rearrange_transfers(bd.transfer_to_compute_map, bd.label_to_block_id, stats)
            strategy = remap_strategy(strategy, remapped)
            bd = BlockStrategyData(
                label_to_size_map={remapped.get(k, k): v for k, v in bd.label_to_size_map.items()},
                allocation_ordered=create_allocation_ordered(l2b, stats),
                block_sizes=bd.block_sizes,
                label_to_block_id=l2b,
                transfer_to_compute_map=t2c,
            )
        return StreamPlan(streamed, resident, bd, strategy, reordered, budget, gpu, enc)

    def streamed_bytes(p: StreamPlan) -> int:
        return sum(by_label[x].nbytes for x in p.streamed)

    for k in range(1, n + 1):
        plan = attempt(k)
        if plan is None:
            continue
        if not encodable or budget is None:
            return plan
        # Units kept encoded make room by bytes, not by count: among the counts up to twice the first
        # that fits, the plan that streams the fewest bytes (ties: fewer units).
        for more in range(k + 1, min(n, 2 * k) + 1):
            other = attempt(more)
            if other is not None and streamed_bytes(other) < streamed_bytes(plan):
                plan = other
        return plan
    # Even streaming every unit does not fit: the tensors placed outside the
    # units leave too little for the ring (gpu_budget.py:200-225).
    raise RuntimeError(
        "Insufficient GPU budget after reserving the tensors kept on the GPU outside the offload units: "
        f"budget={budget} bytes, reserved_outside_units={base_bytes} bytes, "
        f"effective_budget={max(0, (budget or 0) - base_bytes)} bytes, "
        f"minimum_ring={2 * max(sizes)} bytes (two slots of the largest unit). Raise max_gpu_mem_bytes / "
        "max_gpu_mem_fraction or include the large outside tensors' modules in the offload units.")


def state_from_plan(model: nn.Module, units: Sequence[_Unit], plan: StreamPlan, durations: dict[str, float],
                    loader_type: str, link: LinkMeasurement | None = None) -> TensorManagerState:
    """A plan as a saved state (state_handler.py:501-633): ids are this process's, names tie them to the model.

    ``units`` are the offload units in execution order; ``durations`` their
    profiled seconds. With ``link`` (the measured host link), every tensor's
    ``load_time_ms`` is its size on the measured SDMA curve, the reference's
    per-tensor transfer benchmark (tensor_processors.py:1019-1062) from which a
    loaded profile rebuilds the curve (collectors.py:33-66), and the chosen
    copy policy is saved beside the plan.
    """
    id_to_name = {id(p): n for n, p in model.named_parameters()}
    params = {id(p): p for p in model.parameters()}
    bd = plan.block_data
    interp = MemoryTransferInterpolator(link.memory_transfer_stats()) if link and link.sdma.best_ms else None

    def timed(ts: Sequence[TensorStatistics]) -> list[TensorStatistics]:
        if interp is None:
            return list(ts)
        return [dataclasses.replace(t, load_time_ms=interp.bytes_to_duration(t.size_bytes)) if t.size_bytes else t
                for t in ts]

    strategy = {k: timed(v) for k, v in plan.strategy_map.items()}
    streamed = [t for ts in strategy.values() for t in ts]
    stats = []
    for u in units:
        st = u.stats(durations.get(u.label, 0.0))
        stats.append(dataclasses.replace(st, tensors=timed(st.tensors)))
    return TensorManagerState(
        loader_type=loader_type,
        tensor_id_to_name_map=id_to_name,
        allocation_ordered={b: list(v) for b, v in bd.allocation_ordered.items()} if bd else {},
        label_to_size_map=dict(bd.label_to_size_map) if bd else {},
        block_sizes=dict(bd.block_sizes) if bd else {},
        load_strategy=strategy,
        release_strategy={},
        label_to_block_id=dict(bd.label_to_block_id) if bd else {},
        stats=stats,
        transfer_to_compute_map=dict(bd.transfer_to_compute_map) if bd else {},
        view_tensors_ids=[t.tensor_id for t in streamed],
        view_tensors_names=[t.name for t in streamed],
        gpu_tensors_names=sorted(set(id_to_name.values()) - {t.name for t in streamed}),
        managed_tensor_dtypes={t.name: str(params[t.tensor_id].dtype).removeprefix("torch.") for t in streamed},
        managed_tensor_layouts={t.name: {"shape": list(params[t.tensor_id].shape),
                                         "stride": list(params[t.tensor_id].stride())} for t in streamed},
        copy_policy=link.to_dict() if link is not None else None,
    )


def plan_from_state(state: TensorManagerState, units: Sequence[_Unit], base_bytes: int,
                    budget: int | None, encodable: Mapping[str, tuple[int, int]] | None = None) -> StreamPlan:
    """The saved plan re-keyed to the live tensors by name (the role of state_handler.py:673-745, 1072-1420).

    ``units`` are the live offload units in the saved execution order. A
    streamed tensor that is missing, or whose size, dtype or layout differs
    from the saved metadata, raises ``ValueError``. With ``encodable``, residents
    that do not fit the budget raw are kept encoded in HBM as
    :func:`plan_streaming` keeps them.
    """
    by_name = {n: p for u in units for n, p in zip(u.names, u.params)}
    strategy: dict[str, list[TensorStatistics]] = {}
    for label, ts in state.load_strategy.items():
        cur = []
        for t in ts:
            p = by_name.get(t.name)
            if p is None or p.numel() * p.element_size() != t.size_bytes:
                raise ValueError(f"profile tensor {t.name!r} is missing or has a different size in this model")
            dt = state.managed_tensor_dtypes.get(t.name)
            if dt is not None and str(p.dtype).removeprefix("torch.") != dt:
                raise ValueError(f"profile tensor {t.name!r} was {dt}, the model holds {p.dtype}")
            lay = state.managed_tensor_layouts.get(t.name)
            if lay is not None and (list(p.shape) != lay["shape"] or list(p.stride()) != lay["stride"]):
                raise ValueError(f"profile tensor {t.name!r} has shape/stride {lay['shape']}/{lay['stride']}, "
                                 f"the model holds {list(p.shape)}/{list(p.stride())}")
            cur.append(TensorStatistics(id(p), t.name, t.size_bytes, t.load_time_ms))
        strategy[label] = cur
    bd = state.block_data() if state.load_strategy else None
    order = [u.label for u in units]
    consumers = set(state.transfer_to_compute_map.values())
    streamed = [x for x in order if x in consumers]
    resident = [x for x in order if x not in consumers]
    nxt = {a: order[(i + 1) % len(order)] for i, a in enumerate(order)}
    reordered = any(nxt.get(t) != c for t, c in state.transfer_to_compute_map.items())
    by_label = {u.label: u for u in units}
    ring = sum(bd.block_sizes.values()) if bd else 0
    gpu = base_bytes + sum(by_label[x].nbytes for x in resident) + ring
    enc: dict[str, int] = {}
    if budget is not None and encodable and bd is not None and gpu > budget:
        got = encode_residents(resident, {x: by_label[x].nbytes for x in resident}, encodable,
                               budget - base_bytes - ring)
        if got is not None:
            enc, gpu = got[0], base_bytes + got[1] + ring
    return StreamPlan(streamed, resident, bd, strategy, reordered, budget, gpu, enc)


# Attributes every nn.Module gets from its constructor (parameters, buffers,
# children, hooks); anything else in a module's __dict__ belongs to the model.
_MODULE_INTERNALS = frozenset(vars(nn.Module()))


def plain_tensors(model: nn.Module) -> list[torch.Tensor]:
    """Tensors the model reaches that are neither parameters nor buffers.

    These are plain tensor attributes of its modules and tensors held in lists,
    tuples, sets, dicts or plain objects under them. They go to the GPU like
    the reference's unmapped tensors (tensor_processors.py:324-360,685-742).
    The walk reads and never rebinds. Types, Python module objects and
    nn.Modules are not entered; every module is visited through
    ``model.modules()``. Each object is visited once, so cycles end. Returns
    each tensor once, in first-seen order.
    """
    skip = (type, types.ModuleType, nn.Module, str, bytes, int, float, complex, bool, type(None))
    registered = {id(t) for t in model.parameters()} | {id(t) for t in model.buffers()}
    found: dict[int, torch.Tensor] = {}
    seen: set[int] = set()
    for module in model.modules():
        stack = [v for k, v in reversed(list(vars(module).items())) if k not in _MODULE_INTERNALS]
        while stack:
            value = stack.pop()
            if isinstance(value, torch.Tensor):
                if id(value) not in registered:
                    found.setdefault(id(value), value)
                continue
            if isinstance(value, skip) or id(value) in seen:
                continue
            seen.add(id(value))
            if isinstance(value, dict):
                stack.extend(reversed(list(value.values())))
            elif isinstance(value, (list, tuple)):
                stack.extend(reversed(value))
            elif isinstance(value, (set, frozenset)):
                stack.extend(value)
            elif getattr(type(value), "__dictoffset__", 0) != 0:
                try:
                    stack.extend(reversed(list(vars(value).values())))
                except TypeError:
                    pass
    return list(found.values())


def shared_unit_parameters(model: nn.Module, labels: Sequence[str]) -> dict[int, list[str]]:
    """Parameters that the modules of two or more offload units hold (tied weights): id -> unit labels.

    A streamed parameter lives in its unit's ring slot only while that unit
    runs, so a parameter another unit also reads would be read from a slot the
    ring has since refilled. The reference promotes such cross-layer tensors to
    permanent GPU residence (tensor_manager.py:226-272); these do the same.
    """
    owners: dict[int, list[str]] = {}
    for label in labels:
        mod = _submodule(model, label)
        if mod is None:
            continue
        for pid in {id(q) for q in mod.parameters()}:
            owners.setdefault(pid, []).append(label)
    return {pid: units for pid, units in owners.items() if len(units) > 1}


@contextlib.contextmanager
def _oom_context(tensors: Sequence[torch.Tensor], what: str, advice: str) -> Iterator[None]:
    """Re-raise a device allocation failure naming what was being placed (tensor_manager.py:755-775)."""
    try:
        yield
    except (torch.cuda.OutOfMemoryError, nat.FtxOutOfMemoryError) as exc:
        nbytes = sum(t.numel() * t.element_size() for t in tensors)
        raise torch.cuda.OutOfMemoryError(f"GPU out of memory while moving {len(tensors)} {what} "
                                          f"({nbytes / 2**30:.2f} GiB) to the GPU. {advice}") from exc


def _submodule(model: nn.Module, label: str) -> nn.Module | None:
    if not label:
        return None
    try:
        return model.get_submodule(label)
    except AttributeError:
        return None


class OffloadManager:
    """One named offload session: phases, plan, loader and the patched model."""

    def __init__(self, name: str = DEFAULT_MANAGER_NAME) -> None:
        self.name = name
        self.phase = OffloadPhase.NOT_INITIALIZED
        self.config = OffloadConfig()
        self.model: nn.Module | None = None
        self.device = torch.device("cpu")
        self.units: list[_Unit] = []
        self.order: list[str] = []
        self.durations: dict[str, list[float]] = {}
        self.loader: Any = None
        self.controller: Any = None
        self.plan: StreamPlan | None = None
        self.timing: OffloadTimingCollector | None = None
        self._owner = threading.get_ident()
        self._forwards = 0
        self._hooks: list[Any] = []
        self._patched: list[tuple[nn.Module, Any]] = []
        self._resident_bytes = 0
        self._plain: list[torch.Tensor] = []  # plain tensors moved to the GPU by offload(); release() returns them
        self._cpu_data: dict[int, torch.Tensor] = {}
        self._seen_this_pass: list[str] = []
        self._events: dict[str, tuple[Any, Any]] = {}
        self._pass_done: list[Any] = []  # completion events of the latest streamed passes
        self.build_seconds = 0.0
        self.compile_fn: Callable[[nn.Module], Any] | None = None
        self._load_from_shm = False
        self._suspend_count = 0  # profiling suspensions outstanding (reference-counted)
        # what init()/offload() set up: None before either, "noop" for enabled=False, else "live"
        self._control: str | None = None
        self._from_state = False
        self._reload_pending = False
        self._hbm_keys: dict[str, str] = {}  # unit label -> its block key, for units kept encoded in HBM
        self._stale_encoding: str | None = None  # why the encoded blocks no longer match the model's weights
        self._pinner: HostPinner | None = None
        self.memory_transfer_stats: dict[int, float] = {}
        self.link: LinkMeasurement | None = None  # the measured host link and the copy policy it chose
        self._reset_replan()
        self.skip_discovery_honored: bool | None = None  # None until offload() decides
        self._discovery_passes = 0
        self._reset_manual()

    def _reset_manual(self) -> None:
        self._manual = False  # no module units: manual offload blocks, parameters placed on first use
        self._pending: dict[int, nn.Parameter] = {}  # parameters still on the host, not yet placed for good
        self._block_owner: dict[int, str] = {}
        self._block_params: dict[str, list[nn.Parameter]] = {}
        self._empty_blocks: set[str] = set()
        self._block: str | None = None  # the manual block being run
        self._block_tmp: list[nn.Parameter] = []
        self._mode_depth = 0
        self._mode: _DiscoveryMode | None = None
        self._quiet = False  # set while the manager itself moves parameters under the discovery mode

    # -- public ---------------------------------------------------------------

    def offload(self, model: nn.Module, config: OffloadConfig | None = None,
                state: TensorManagerState | None = None,
                compile_fn: Callable[[nn.Module], Any] | None = None, *,
                load_from_shm: bool = False) -> nn.Module:
        """Patch ``model``; with a saved ``state`` the plan is restored and streaming starts at once.

        ``compile_fn`` is the reference's per-unit compiler (offload_manager.py:2858-2884): at the
        INFERENCE transition it is applied to each offload unit, so every unit compiles as its own
        graph with the unit's ``pre_compute`` / ``post_compute`` ops inside. Discovery and
        profiling stay eager.
        """
        self._check_thread()
        if self.model is not None:
            raise RuntimeError(f"offload manager {self.name!r} already manages a model; release() it first")
        if compile_fn is not None and not callable(compile_fn):
            raise TypeError("compile_fn must be callable: module -> compiled module")
        self.config = config or OffloadConfig()
        if load_from_shm and (state is None or not self.config.shm_enabled or not state.shm_block_name_map):
            raise ValueError("load_from_shm needs shm_enabled and a saved state that names its shared blocks")
        if self.config.enabled and self.config.pinned_memory and self.config.pinned_memory_mode == "host_register":
            raise ValueError(nat.HOST_REGISTER_REFUSED)
        self.compile_fn = compile_fn
        self._load_from_shm = load_from_shm
        self._control = "live" if self.config.enabled else "noop"
        if not self.config.enabled:
            return model
        nat.load()
        name_of = {id(p): n for n, p in model.named_parameters()}
        if state is not None:
            labels = [s.label for s in state.stats]
            self._check_state(state, name_of)
        else:
            labels = select_offload_units(model, self.config.include_patterns, self.config.exclude_patterns)
        units: list[_Unit] = []
        unit_params: set[int] = set()
        by_name = dict(model.named_parameters())
        saved = {st.label: [t.name for t in st.tensors] for st in state.stats} if state is not None else {}
        shared = shared_unit_parameters(model, labels)
        if shared:
            mib = sum(by_name[name_of[pid]].numel() * by_name[name_of[pid]].element_size() for pid in shared) / 2**20
            LOGGER.warning("offload %r: %d parameter(s) belong to more than one offload unit and stay on the GPU for "
                           "good (offload coverage reduced by %.2f MiB): %s", self.name, len(shared), mib,
                           ", ".join(f"{name_of[pid]} ({' + '.join(u)})" for pid, u in list(shared.items())[:8]))
        streamed = parameter_filter(model, self.config.include_patterns, self.config.exclude_patterns)
        for label in labels:
            mod = _submodule(model, label)
            params = []
            if mod is not None:
                kept = [(n, q) for n, q in mod.named_parameters() if id(q) not in unit_params and id(q) not in shared]
                params = [q for n, q in kept if streamed(f"{label}.{n}")]
                if kept and not params and state is None:
                    LOGGER.warning("offload %r: include/exclude patterns leave unit %r no parameter to stream; its "
                                   "parameters stay on the GPU", self.name, label)
            names = [name_of[id(p)] for p in params]
            if state is not None and mod is not None and names != saved[label]:
                own = {name_of[id(q)] for q in mod.parameters() if id(q) not in shared}
                if set(saved[label]) <= own:
                    # the saved profile decides what the unit streams, over the runtime patterns, as the
                    # reference adopts a profile's strategy; the module's other parameters stay resident
                    names = list(saved[label])
                    params = [by_name[n] for n in names]
                elif self.config.include_patterns:
                    # a module unit would stream tensors outside its module, which other modules may read
                    # while its slot holds another unit
                    raise ValueError(f"profile unit {label!r} streams {saved[label]}, which are not all parameters "
                                     f"of the module {label!r} (tied or elsewhere in the model); profile this model "
                                     "again")
            if state is not None and (mod is None or names != saved[label]):
                # a manual offload block of the saved plan: its tensors by name
                mod = None
                names = [n for n in saved[label] if n in by_name and id(by_name[n]) not in unit_params]
                params = [by_name[n] for n in names]
            unit_params.update(id(p) for p in params)
            units.append(_Unit(label, mod, params, names))
        if state is not None:
            plan_from_state(state, units, 0, None)  # every mismatch surfaces before the model is touched
        for setting in self.config.inert_settings():
            LOGGER.warning("offload %r: %s has no effect in this build (it steers the reference's strategy search "
                           "or instrumentation)", self.name, setting)
        self._from_state = state is not None
        self.skip_discovery_honored = None
        if state is None and self.config.skip_discovery:
            self.skip_discovery_honored = bool(units)
            if not units:
                LOGGER.warning("offload %r: skip_discovery=True but include_patterns select no module; running the "
                               "discovery passes instead", self.name)
        self._discovery_passes = 0 if self.skip_discovery_honored else self.config.discovery_iters
        self.device = torch.device("cuda", self.config.gpu_device)
        torch.cuda.set_device(self.device)
        self.model = model
        self.units = units
        try:
            self._manual = state is None and not units and self._discovery_passes > 0
            if self._manual:
                # manual offload blocks: parameters wait on the host until discovery sees where they are used
                self._pending = {id(p): p for p in model.parameters() if p.device.type == "cpu"}
                self._plain = [t for t in plain_tensors(model) if t.device.type == "cpu"]
                self._resident_bytes += self._upload_into([b for b in model.buffers() if b.device.type == "cpu"]
                                                          + self._plain)
                self._patch_root(model)
            else:
                self._place_outside_units(unit_params)
            custom_ops.register_manager(id(self), self)
            for u in self.units:
                if u.module is not None:
                    self._patch(u)
            # first in line (offload_manager.py:2214-2242): the manager opens each pass before any user
            # pre-hook runs, and user forward hooks see the phase this pass moved to
            self._hooks.append(model.register_forward_pre_hook(lambda *_: self._before_forward(), prepend=True))
            self._hooks.append(model.register_forward_hook(lambda *_: self._after_forward(), prepend=True))
            self.phase = OffloadPhase.DISCOVERY if self._discovery_passes > 0 else OffloadPhase.PROFILING
            if state is not None:
                self.order = labels
                self._to_inference(state)
            elif self.config.discovery_iters == 0 and self.config.profiling_iters == 0:
                self.order = [u.label for u in self.units]
                self._to_inference()
        except BaseException:
            self._abandon()
            raise
        return model

    def _release_pins(self) -> None:
        """End the in-place page locks of ``host_register`` mode (host_pinning.py:314-344).

        The reference releases pins at manager shutdown, not with the blocks.
        The memory stays valid, now pageable, for the views that still hold it.
        """
        pinner, self._pinner = self._pinner, None
        if pinner is not None:
            pinner.release_all()

    def _abandon(self) -> None:
        """Undo the manager's own changes after a failed ``offload()`` so it can be used again
        (offload_manager.py:1932-1937): hooks, patched forwards and the loader go; tensors
        already placed on the GPU stay there, so the model should be discarded."""
        for h in self._hooks:
            h.remove()
        self._unpatch(self._patched)
        if self._mode is not None:
            self._mode_depth = 1
            self._pop_mode()
        custom_ops.unregister_manager(id(self))
        if self.loader is not None:
            try:
                self.loader.shutdown()
            except Exception:  # noqa: BLE001 - the primary error is the one to report
                LOGGER.exception("offload %r: loader shutdown after a failed offload() failed", self.name)
        self._reset_manual()
        self._release_pins()
        self.loader = self.controller = self.plan = self.timing = None
        self.link = None
        self._reset_replan()
        self.model = None
        self.units, self._patched, self._hooks, self.order = [], [], [], []
        self._seen_this_pass, self._pass_done, self._events = [], [], {}
        self._cpu_data = {}
        self._forwards = 0
        self._resident_bytes = 0
        self._plain = []
        self._control, self._suspend_count = None, 0
        self._from_state = False
        self._reload_pending = False
        self._hbm_keys, self._stale_encoding = {}, None
        self.skip_discovery_honored = None
        self.compile_fn = None
        self._load_from_shm = False
        self.phase = OffloadPhase.NOT_INITIALIZED

    def _check_state(self, state: TensorManagerState, name_of: dict[int, str]) -> None:
        if state.loader_type != self.config.transfer_mode:
            raise ValueError(f"profile was made with transfer_mode={state.loader_type!r}, "
                             f"config selects {self.config.transfer_mode!r}")
        self._check_inventory(state, name_of)

    def _check_inventory(self, state: TensorManagerState, name_of: dict[int, str]) -> None:
        saved = set(state.tensor_id_to_name_map.values())
        current = set(name_of.values())
        if saved != current:
            raise ValueError(f"profile does not match the model: missing={sorted(saved - current)[:8]}, "
                             f"unexpected={sorted(current - saved)[:8]}")

    def _resolve_profile_directory(self, profile_directory: str | None) -> str:
        """The explicit directory, else ``config.profile_storage_dir`` (offload_manager.py:750-768)."""
        resolved = profile_directory or (self.config.profile_storage_dir if self.config is not None else None)
        if resolved is None:
            raise ValueError("No profile directory specified. Provide profile_directory argument "
                             "or set profile_storage_dir in OffloadConfig.")
        return resolved

    def save_profile(self, profile_directory: str | None = None) -> str:
        """Write the current plan as ``<dir>/profile.json`` (schema 3); returns the file path.

        Mirrors offload_manager.py:770-792: a manager with no model raises
        ``RuntimeError``; a missing directory raises ``ValueError``.
        """
        if self.config.profile_read_only:
            raise ValueError("Cannot save profile: config.profile_read_only is True. "
                             "Set profile_read_only=False in OffloadConfig to enable saving.")
        if self.model is None:
            raise RuntimeError("Tensor manager not initialized. Call offload() first.")
        directory = self._resolve_profile_directory(profile_directory)
        if self.phase != OffloadPhase.INFERENCE or self.plan is None:
            raise RuntimeError("No profile data yet: the model has not reached the INFERENCE phase.")
        return str(save_state(self.state(), directory))

    def load_profile(self, profile_directory: str | None = None, model: nn.Module | None = None) -> None:
        """Adopt ``<dir>/profile.json`` (offload_manager.py:794-816).

        With no model under management, ``model`` is offloaded with the saved
        plan. A model still in discovery or profiling switches to streaming
        with the saved plan at once.
        """
        self._check_thread()
        target = model if model is not None else self.model
        if target is None:
            raise RuntimeError("No model provided and no model has been offloaded yet.")
        state = load_state(self._resolve_profile_directory(profile_directory))
        if self.model is None:
            self.offload(target, self.config, state=state)
            return
        if target is not self.model:
            raise RuntimeError("this manager manages another model; release() it first")
        if self.phase == OffloadPhase.INFERENCE:
            raise RuntimeError("the model is already streaming; release() it before loading a profile")
        self._check_state(state, {id(p): n for n, p in self.model.named_parameters()})
        saved = [s.label for s in state.stats]
        if set(saved) != {u.label for u in self.units}:
            diff = sorted(set(saved) ^ {u.label for u in self.units})
            raise ValueError(f"profile offload units differ from this model's: {diff[:8]}")
        plan_from_state(state, [self._unit(x) for x in saved], 0, None)  # mismatches raise before any change
        self.order = saved
        self._to_inference(state)

    def state(self) -> TensorManagerState:
        """The plan as a :class:`TensorManagerState` keyed by this process's tensor ids."""
        assert self.model is not None and self.plan is not None
        state = state_from_plan(self.model, [self._unit(x) for x in self.order], self.plan,
                                {x: self._duration(x) for x in self.order}, self.config.transfer_mode, self.link)
        names = getattr(self.controller, "shm_block_name_map", None)
        if names:
            state.shm_block_name_map = dict(names)
        return state

    def _duration(self, label: str) -> float:
        d = self.durations.get(label, [])
        return float(sum(d) / len(d)) if d else 0.0

    @property
    def iters_before_inference(self) -> int:
        """Forwards that take the offloaded model to INFERENCE (offload_manager.py:1827-1863).

        Discovery passes count unless they are skipped (``skip_discovery``
        honoured, or ``discovery_iters=0``). A skipped discovery still takes one
        profiling forward, which records the execution order. A model offloaded
        with a saved plan streams at once (0).
        """
        if self.model is None or self._from_state:
            return 0
        d, p = self.config.discovery_iters, self.config.profiling_iters
        if d == 0 and p == 0:
            return 0
        if self.skip_discovery_honored:
            return max(1, p)
        return d + p

    def get_gpu_memory_usage(self) -> GPUMemoryUsage:
        """Ring-slot and permanently placed bytes; only in INFERENCE (offload_manager.py:866-905)."""
        if self.phase != OffloadPhase.INFERENCE:
            raise RuntimeError(f"Cannot get GPU memory usage in phase {self.phase.value}. "
                               "This method is only available after transitioning to inference mode.")
        blocks = self.loader.get_gpu_memory_bytes() if self.loader is not None else 0
        return GPUMemoryUsage(blocks, self._resident_bytes)

    def collect_offload_timing(self) -> OffloadTimingReport | None:
        return self.timing.report() if self.timing is not None and self.timing.enabled else None

    def reset_offload_timing(self) -> None:
        if self.timing is not None:
            self.timing.reset()

    def reset_offload_timing_sampling(self) -> None:
        """Drop the stored timing passes and close the sample window (offload_manager.py:1439-1444).

        From then on only passes between :meth:`begin_offload_timing_sample`
        and :meth:`finish_offload_timing_sample` are stored.
        """
        self.reset_offload_timing()
        if self.timing is not None:
            self.timing.set_measure_window(False)

    def begin_offload_timing_sample(self) -> None:
        """Open the sample window for the next pass (offload_manager.py:1446-1450)."""
        if self.timing is not None:
            self.timing.set_measure_window(True)

    def finish_offload_timing_sample(self, *, replay_generation: int | None) -> bool:
        """Store the sampled pass, then close the window; True if one was stored (offload_manager.py:1452-1463).

        ``replay_generation`` is None for an eager pass. For a graph replay
        the latest replay is read: the timestamps here are rewritten by every
        replay, so no generation needs matching.
        """
        if self.timing is None or not self.timing.enabled:
            return False
        try:
            return self.timing.flush()
        finally:
            self.timing.set_measure_window(False)

    def cancel_offload_timing_sample(self) -> None:
        """Close the sample window without storing (offload_manager.py:1465-1469)."""
        if self.timing is not None:
            self.timing.set_measure_window(False)

    def sync_prev_onload(self) -> None:
        """Make the current stream wait for the transfers issued so far (offload_manager.py:858-860)."""
        fn = getattr(self.loader, "sync_prev_onload", None)
        if fn is not None:
            fn()

    def join_after_forward(self) -> None:
        """Join the transfer stream back into the current one after a forward (offload_manager.py:862-864)."""
        fn = getattr(self.loader, "join_after_forward", None)
        if fn is not None:
            fn()

    def get_layer_label_by_idx(self) -> list[str]:
        """Labels of the patched module units, in patch order (offload_manager.py:1203-1214)."""
        return [u.label for u in self.units if u.module is not None]

    @property
    def eager_profiling_iters(self) -> int:
        """Profiling forwards before INFERENCE, at least 1 (offload_manager.py:731-740)."""
        return max(1, self.config.profiling_iters)

    def get_memory_transfer_stats(self) -> dict[int, float] | None:
        """The measured host-link curve ``{bytes: ms}`` (SDMA) of the current plan, None before INFERENCE
        (tensor_manager.py:1632-1639)."""
        return dict(self.memory_transfer_stats) if self.memory_transfer_stats else None

    def benchmark_transfers(self) -> dict[int, float]:
        """Measure host-to-device copy times at the largest unit's size and below
        (memory_transfer_benchmark.py:59-129); returns and keeps ``{bytes: ms}``.

        The reference's method of this name is an empty placeholder
        (offload_manager.py:844-848).
        """
        if self.model is None:
            return {}
        largest = max((u.nbytes for u in self.units), default=0)
        if largest == 0:
            return {}
        from .link_model import benchmark_memory_transfers

        self.memory_transfer_stats = benchmark_memory_transfers(largest, self.device)
        return self.memory_transfer_stats

    def offload_from_state(self, model: nn.Module, state: TensorManagerState, config: OffloadConfig | None = None,
                           *, allow_strategy_replan: bool = True) -> nn.Module:
        """Adopt a saved plan (offload_manager.py:1924-1960): streaming starts at the first forward.

        ``allow_strategy_replan`` is accepted for the reference's signature;
        there is no strategy replan here.
        """
        if self.phase != OffloadPhase.NOT_INITIALIZED or self.model is not None:
            raise RuntimeError("OffloadManager is already active; call release() before adopting another state.")
        return self.offload(model, config if config is not None else self.config, state=state)

    def init(self, config: OffloadConfig | None = None) -> None:
        """Set the configuration before ``offload`` (offload_manager.py:2853-2856)."""
        self.set_config(config or OffloadConfig())
        self._control = "live" if self.config.enabled else "noop"

    def set_config(self, config: OffloadConfig) -> None:
        """Replace the configuration; refused once a model is managed (offload_manager.py:2887-2895)."""
        self._check_thread()
        if self.model is not None:
            raise RuntimeError(f"offload manager {self.name!r} already manages a model; release() it before "
                               "changing its configuration")
        self.config = config

    def offload_units(self) -> tuple[tuple[str, nn.Module], ...]:
        """The patched offload units as ``(qualified_name, live module)`` pairs, in selection order
        (offload_manager.py:1216-1238).

        The module is the one at that path now, so a unit the caller replaced
        (a compiled wrapper) is returned as the replacement. Paths that no
        longer resolve are skipped; a module reachable by two units is listed
        once. Manual ``offload_block`` regions have no module and are not
        listed. Which of them stream is ``plan.streamed``.
        """
        if self.model is None:
            return ()
        seen: set[int] = set()
        out: list[tuple[str, nn.Module]] = []
        for u in self.units:
            if u.module is None:
                continue
            try:
                live = self.model.get_submodule(u.label)
            except (AttributeError, KeyError):
                continue
            if id(live) not in seen:
                seen.add(id(live))
                out.append((u.label, live))
        return tuple(out)

    def resident_units(self) -> tuple[tuple[str, nn.Module], ...]:
        """The outermost modules that are not offload units and contain none (offload_manager.py:1240-1265;
        compile/module_swap.py:105-160): the parts of the model that stay on the GPU.

        The root is never listed. A module holding an offload unit, or a
        container without a forward of its own (``ModuleList``,
        ``ModuleDict``), is descended into; children of offload units are
        omitted; a shared module is listed once, at its first path.
        """
        if self.model is None:
            return ()
        offload_ids = {id(m) for _, m in self.offload_units()}
        holds: dict[int, bool] = {}

        def holds_unit(mod: nn.Module) -> bool:
            key = id(mod)
            if key not in holds:
                holds[key] = False  # a module tree with a cycle stops here
                holds[key] = key in offload_ids or any(holds_unit(c) for c in mod.children())
            return holds[key]

        out: list[tuple[str, nn.Module]] = []
        seen: set[int] = set()

        def visit(path: str, mod: nn.Module, root: bool) -> None:
            if not root and id(mod) in offload_ids:
                return
            if root or holds_unit(mod) or type(mod).forward is nn.Module.forward:
                for name, child in mod.named_children():
                    visit(f"{path}.{name}" if path else name, child, False)
                return
            if id(mod) not in seen:
                seen.add(id(mod))
                out.append((path, mod))

        visit("", self.model, True)
        return tuple(out)

    def _profiling_control(self, what: str) -> bool:
        """Whether profiling control acts: refused before ``init``/``offload``, inert for a disabled
        offload, as the reference's no-op manager (offload_manager.py:2521-2620)."""
        if self._control is None:
            raise RuntimeError(f"{what}() called before flextensor.offload(...); call flextensor.offload(model, "
                               "config=...) first.")
        return self._control == "live"

    def clear_profiling_durations(self) -> None:
        """Drop every profiled duration; the unit order found by discovery stays (offload_manager.py:3131-3141)."""
        if self._profiling_control("clear_profiling_durations"):
            self.durations.clear()

    def suspend_profiling(self) -> None:
        """Stop recording profiling passes until the matching :meth:`resume_profiling`.

        Suspensions nest. A suspended profiling pass records no durations and
        does not count against ``profiling_iters`` (offload_manager.py:3144-3184).
        """
        if self._profiling_control("suspend_profiling"):
            self._suspend_count += 1

    def resume_profiling(self) -> None:
        if not self._profiling_control("resume_profiling"):
            return
        if self._suspend_count == 0:
            raise RuntimeError("resume_profiling() without a matching suspend_profiling()")
        self._suspend_count -= 1

    def is_profiling_suspended(self) -> bool:
        """Whether a suspension is outstanding; always False for a disabled offload."""
        return self._control == "live" and self._suspend_count > 0

    @contextlib.contextmanager
    def pause_profiling(self) -> Iterator[None]:
        """Context-manager form of suspend/resume (offload_manager.py:3199-3220)."""
        if not self._profiling_control("pause_profiling"):
            yield
            return
        self.suspend_profiling()
        try:
            yield
        finally:
            self.resume_profiling()

    def update_state(self) -> None:
        """Advance the phase machine by one pass, as the post-forward hook does (offload_manager.py:3110-3123).

        For passes the hook does not see, such as graph replays.
        """
        self._after_forward()

    # ---- re-measuring the plan in flight (offload_manager.py:667-720, 1294-1325) ----------------------------

    def _reset_replan(self) -> None:
        self._replan: dict[str, Any] | None = None  # the armed tail: passes left, its collector, its start
        self._replan_state: StrategyReplanState = "idle"
        self._replan_applied: bool | None = None

    def _strategy_replan_unavailable_reason(self, manual: bool = False) -> str | None:
        """Why a replan request cannot start now, or None when it can."""
        if self.phase != OffloadPhase.INFERENCE:
            return (f"the offload is in {self.phase.value}; run iters_before_inference forwards to reach "
                    "inference first")
        if self._replan is not None:
            return "a replan is already in flight; run the passes the request returned"
        if self._replan_state == "failed":
            return "an earlier replan failed, so inference is already unsafe; release the model and offload it again"
        if self.controller is None or self.loader is None:
            return "nothing streams, so there is nothing to re-measure"
        if hip.is_capturing():
            return "a graph is being captured"
        if manual and not (self.timing is not None and self.timing.enabled and self.timing.graph_replay):
            return ("manual_update_state=True measures graph replays, which needs offload_timing='cuda_graph' "
                    "when the graph is captured")
        return None

    @property
    def strategy_replan_status(self) -> StrategyReplanStatus:
        """Passive snapshot of the replan; reading it never starts or advances one."""
        applied = self._replan_applied if self._replan_state in ("done", "failed") else None
        return StrategyReplanStatus(self._replan_state, self._strategy_replan_unavailable_reason() is None, applied)

    def _new_replan_collector(self) -> OffloadTimingCollector:
        return OffloadTimingCollector(list(self.order), log_every=0)

    def request_strategy_replan(self, *, manual_update_state: bool = False) -> int:
        """Re-measure the units' compute under the current runtime and rebuild what depends on it.

        What depends on it here is the ring's copy engine: a pass computing
        far less than its streamed units take on the link copies every slot
        with the zero-copy kernel, any other keeps the per-size policy. Call
        it after the compute changed under a running offload (a compiled
        forward, a captured graph, other batch shapes).

        * ``manual_update_state=False``: run the returned number of forwards;
          the post-forward hook advances the replan.
        * ``manual_update_state=True``: for graph replays, which run no hooks.
          Capture with ``offload_timing="cuda_graph"``, then call
          ``graph.replay()`` and :meth:`update_state` the returned number of
          times; recapture afterwards, since the captured copies keep the old
          engine.

        Returns the passes to run (a warm-up pass and the measured ones), or 0
        with a warning when a replan cannot start now
        (:attr:`strategy_replan_status`.can_request).
        """
        self._check_thread()
        reason = self._strategy_replan_unavailable_reason(manual_update_state)
        if reason is not None:
            LOGGER.warning("offload %r: request_strategy_replan() ignored - %s", self.name, reason)
            return 0
        passes = REPLAN_WARMUP_PASSES + REPLAN_MEASURE_PASSES
        if manual_update_state:
            self._replan = {"left": passes, "manual": True, "start": len(self.timing.snapshots)}
        else:
            # a collector of its own on the loader for these passes: they are timed for the replan and are not
            # reported by collect_offload_timing()
            collector = self._new_replan_collector()
            self._replan = {"left": passes, "manual": False, "collector": collector,
                            "kept": self.loader.offload_timing_collector}
            self.loader.offload_timing_collector = collector
        self._replan_state, self._replan_applied = "in_progress", None
        LOGGER.info("offload %r: replan armed; run %d passes", self.name, passes)
        return passes

    def _advance_replan(self) -> None:
        tail = self._replan
        if tail is None:
            return
        if tail["manual"]:
            self.timing.flush()  # publishes the latest replay's times
        tail["left"] -= 1
        if tail["left"] > 0:
            return
        self._replan = None
        try:
            if tail["manual"]:
                passes = list(self.timing.snapshots[tail["start"]:])
            else:
                try:
                    passes = list(tail["collector"].report().passes)
                finally:
                    self.loader.offload_timing_collector = tail["kept"]
            self._rebuild_from(passes[-REPLAN_MEASURE_PASSES:])
        except Exception:
            self._replan_state, self._replan_applied = "failed", False
            LOGGER.exception("offload %r: the replan failed; inference is unsafe until the model is offloaded again",
                             self.name)
            raise

    def _rebuild_from(self, passes: list) -> None:
        """New unit durations from the measured passes, and the ring's copy policy re-decided from them."""
        measured = measured_compute(passes, self.order)
        self._replan_state = "done"
        if not measured:
            self._replan_applied = False
            LOGGER.warning("offload %r: the replan measured no unit; the plan is kept", self.name)
            return
        for label, ms in measured.items():
            self.durations[label] = [ms]
        plan = self.plan
        if self.link is None or self.controller is None or plan is None:
            # no link measurement (link_benchmark=False or a pinned copy engine): nothing decided from the times
            self._replan_applied = False
            LOGGER.info("offload %r: replan measured %d units; the copy engine does not depend on them", self.name,
                        len(measured))
            return
        compute_ms = sum(self._duration(x) for x in [*plan.streamed, *plan.resident])
        link = replanned_link(self.link, compute_ms, [self._unit(x).nbytes for x in plan.streamed])
        self.link = link
        self.memory_transfer_stats = link.memory_transfer_stats()
        self.controller.copy_policy = link.native_policy()
        self._apply_link_bound_order()
        self._replan_applied = True
        LOGGER.info("offload %r: replanned: %s", self.name, link.describe())

    def update_offload_timing(self) -> bool:
        """Store the current timing pass (offload_manager.py:3061-3072); True when stored or timing is off."""
        if self.timing is not None and self.timing.enabled:
            self.timing.flush()
        return True

    def release(self, preserve_model: bool = True) -> None:
        """Stop streaming and hand the model back (tensors on the CPU when preserved).

        In the reference's order (tensor_manager.py:2377-2421): the tensors are
        put back first, then the loader shuts down and the in-place pins end.
        A loader that fails to shut down still has the pins released before its
        error is raised again; a pin-release failure on top of it is only
        logged. A transfer stream that cannot be synchronised keeps the pins,
        since a copy may still read them. The manager is reset in every case.
        """
        self._check_thread()
        if self.model is None:
            self._control, self._suspend_count = None, 0
            return
        torch.cuda.synchronize(self.device)
        custom_ops.unregister_manager(id(self))
        for h in self._hooks:
            h.remove()
        self._unpatch(self._patched)
        for u in self.units:
            u.compiled = None
        self.compile_fn = None
        self._load_from_shm = False
        restore: dict[int, torch.Tensor] = {}
        shared: set[int] = set()
        if self.controller is not None and preserve_model:
            for label, block in self.controller.block_map_cpu.items():
                ids = self.controller.label_to_cpu_tensor_id_map[label]
                for tid, view in zip(ids, self._cpu_views(label)):
                    restore[tid] = view
                    if getattr(block, "shm_segment", None) is not None:
                        shared.add(tid)
        params = {id(p): p for u in self.units for p in u.params}
        params.update({id(p): p for p in self.model.parameters()})
        teardown_error: Exception | None = None
        try:
            for tid, p in params.items():
                if not preserve_model:
                    p.data = torch.empty(0, dtype=p.dtype)
                elif tid in restore:
                    # the host block's own view (tensor_manager.py:2320-2354): no second copy of the model;
                    # a shared-memory block is copied out so the parameter does not keep other processes' segment
                    p.data = restore[tid].clone() if tid in shared else restore[tid]
                elif p.device.type != "cpu":
                    p.data = p.data.cpu()
            if preserve_model:
                for b in self.model.buffers():
                    b.data = b.data.cpu()
                for t in self._plain:
                    t.data = t.data.cpu()
            try:
                if self.loader is not None:
                    self.loader.shutdown()
            except TransferStreamSynchronizationError:
                self._pinner = None  # a copy may still read the pinned blocks: their pins stay
                raise
            except Exception as exc:  # noqa: BLE001 - raised again once the pins are released
                teardown_error = exc
            try:
                self._release_pins()
            except Exception:
                if teardown_error is None:
                    raise
                LOGGER.exception("offload %r: host pinner release_all() failed after the loader shutdown failed; "
                                 "the remaining pins stay until the process exits", self.name)
        finally:
            self._plain = []
            self._suspend_count = 0
            self._control = None
            if self._mode is not None:
                self._mode_depth = 1
                self._pop_mode()
            self._reset_manual()
            self._pinner = None
            self._from_state = False
            self._reload_pending = False
            self._hbm_keys, self._stale_encoding = {}, None
            self.skip_discovery_honored = None
            self.loader = self.controller = self.plan = None
            self.link = None
            self._reset_replan()
            self._pass_done = []
            self.model = None
            self.units, self._patched, self._hooks = [], [], []
            self.phase = OffloadPhase.NOT_INITIALIZED
        if teardown_error is not None:
            raise teardown_error

    # -- internals ------------------------------------------------------------

    def _check_thread(self) -> None:
        here = threading.get_ident()
        if here != self._owner:
            raise RuntimeError(f"offload manager {self.name!r} belongs to thread {self._owner} but was used from "
                               f"thread {here}; each named manager is used from the thread that created it")

    def _cpu_views(self, label: str) -> list[torch.Tensor]:
        block = self.controller.block_map_cpu[label]
        if isinstance(self.controller, RawBlockController):
            from .controllers import RawBlockController as R

            return R.reconstruct_original_shapes(block, self.controller.block_meta_map[label])
        return block.views

    def _place_outside_units(self, unit_params: set[int]) -> None:
        """Tensors outside the offload units go to the GPU once (stream-and-scatter): parameters and
        buffers of no unit, and every plain tensor the model reaches (tensor_manager.py:2547-2565)."""
        assert self.model is not None
        rest = [p for p in self.model.parameters() if id(p) not in unit_params and p.device.type == "cpu"]
        bufs = [b for b in self.model.buffers() if b.device.type == "cpu"]
        plain = [t for t in plain_tensors(self.model) if t.device.type == "cpu"]  # never streamed
        self._plain = plain
        with _oom_context(rest + bufs + plain, "tensors outside the offload units", "Tensors outside the offload "
                          "units (not matching include_patterns, or matching exclude_patterns, and tensors that are "
                          "not parameters or buffers) stay on the GPU for good. Broaden include_patterns or narrow "
                          "exclude_patterns."):
            self._resident_bytes += self._upload_into(rest + bufs + plain)

    def _upload_into(self, tensors: Sequence[torch.Tensor]) -> int:
        cpu = [t for t in tensors if t.device.type == "cpu" and t.numel()]
        if not cpu:
            return 0
        dests = upload_tensors([t.data for t in cpu], self.device)
        for t, d in zip(cpu, dests):
            t.data = d
        return sum(t.numel() * t.element_size() for t in cpu)

    # -- manual offload blocks -----------------------------------------------------

    def offload_block(self, name: str) -> OffloadBlock:
        """A context manager that makes the code inside it the offload unit ``name``
        (offload_manager.py:2251-2298).

        For models offloaded with no module units (``include_patterns=[]``).
        Discovery passes record which parameters the block uses; later passes
        load them on entry (profiling) or stream them (inference). A block
        around a module unit that the manager already patches does nothing.
        Blocks run eagerly and do not nest.

        Example::

            with om.offload_block("encoder"):
                out = encoder(hidden)
        """
        self._check_thread()
        if self.model is None:
            raise RuntimeError("Tensor manager not initialized. Call offload() on a model first to initialize the "
                               "manager.")
        if self.skip_discovery_honored:
            raise RuntimeError("offload_block() is not supported when OffloadConfig.skip_discovery is True: manual "
                               "offload blocks are found in the discovery passes. Set skip_discovery=False.")
        return OffloadBlock(self, name)

    def _block_enter(self, label: str) -> str | None:
        """Start block ``label``; returns what its exit must undo (None: nothing)."""
        self._check_thread()
        if self.model is None:
            raise RuntimeError(f"offload manager {self.name!r} manages no model (released?)")
        if torch.compiler.is_compiling():
            raise RuntimeError("offload_block runs eagerly: compile the code inside the block instead")
        if self._block is not None:
            raise RuntimeError(f"offload block {label!r} opened inside block {self._block!r}: blocks do not nest")
        unit = next((u for u in self.units if u.label == label), None)
        if unit is not None and unit.module is not None:
            return None  # a patched module unit traps itself
        if self.phase == OffloadPhase.DISCOVERY:
            if not self._manual:
                raise RuntimeError("manual offload blocks need a model offloaded with no module units "
                                   f"(include_patterns=[]); this model has {len(self.units)} patched unit(s)")
            if label in self._seen_this_pass:
                raise NotImplementedError(f"offload unit {label!r} ran twice in one forward")
            self._seen_this_pass.append(label)
            self._block, self._block_tmp = label, []
            self._push_mode()
            return "discovery"
        if label in self._empty_blocks:
            return None
        if unit is None:
            raise RuntimeError(f"offload block {label!r} was not seen during discovery; every manual block must run "
                               "in the discovery passes (discovery_iters > 0)")
        self._enter(label)
        self._block = label
        return "unit"

    def _block_exit(self, label: str, kind: str) -> None:
        self._block = None
        if kind == "unit":
            self._exit(label)
            return
        self._quiet = True  # the mode must not take these moves for uses of the parameters
        try:
            for p in self._block_tmp:  # uploaded for this block only: back to the host
                if id(p) in self._cpu_data and self._block_owner.get(id(p)) == label:
                    p.data = self._cpu_data.pop(id(p))
        finally:
            self._quiet = False
        self._block_tmp = []
        self._pop_mode()

    def _push_mode(self) -> None:
        if self._mode_depth == 0:
            self._mode = _DiscoveryMode(self)
            self._mode.__enter__()
        self._mode_depth += 1

    def _pop_mode(self) -> None:
        self._mode_depth -= 1
        if self._mode_depth == 0 and self._mode is not None:
            mode, self._mode = self._mode, None
            mode.__exit__(None, None, None)

    def _touch(self, p: nn.Parameter) -> None:
        """Discovery saw ``p`` used: place it for the current block, or on the GPU for good."""
        pid, label = id(p), self._block
        owner = self._block_owner.get(pid)
        if label is not None and owner in (None, label):
            if owner is None:
                self._block_owner[pid] = label
                self._block_params.setdefault(label, []).append(p)
            if pid not in self._cpu_data:
                self._cpu_data[pid] = p.data
                p.data = p.data.to(self.device)
                self._block_tmp.append(p)
            return
        # used outside every block, or by a second block: it stays on the GPU
        if owner is not None:
            del self._block_owner[pid]
            self._block_params[owner] = [q for q in self._block_params[owner] if q is not p]
        del self._pending[pid]
        if self._cpu_data.pop(pid, None) is None:
            p.data = p.data.to(self.device)
        self._resident_bytes += p.numel() * p.element_size()

    def _patch_root(self, model: nn.Module) -> None:
        """Watch the whole forward during manual discovery, so parameters used outside blocks are placed too."""
        own = model.__dict__.get("forward")
        mgr = self

        def forward(self_module: nn.Module, *args: Any, **kwargs: Any) -> Any:
            def orig() -> Any:
                return own(*args, **kwargs) if own is not None else type(self_module).forward(self_module, *args,
                                                                                              **kwargs)

            if mgr.phase == OffloadPhase.DISCOVERY and mgr._pending and not torch.compiler.is_compiling():
                mgr._push_mode()
                try:
                    return orig()
                finally:
                    mgr._pop_mode()
            return orig()

        model.forward = types.MethodType(forward, model)
        self._patched.append((model, own))

    def _finish_manual_discovery(self) -> None:
        """The blocks seen become units; parameters no block owns go to the GPU for good."""
        if not self._manual or self.model is None:
            return
        order = list(self.order) + [x for x in self._block_params if x not in self.order]
        name_of = {id(p): n for n, p in self.model.named_parameters()}
        units = []
        for label in order:
            params = self._block_params.get(label, [])
            if params:
                units.append(_Unit(label, None, list(params), [name_of[id(p)] for p in params]))
            else:
                self._empty_blocks.add(label)
        owned = {id(p) for u in units for p in u.params}
        self._quiet = True
        try:
            self._resident_bytes += self._upload_into([p for pid, p in self._pending.items() if pid not in owned])
        finally:
            self._quiet = False
        self._pending = {}
        self.units = units
        self.order = [u.label for u in units]

    def _patch(self, unit: _Unit) -> None:
        """Wrap the unit's forward in enter/exit (offload_manager.py:1114-1162).

        Eagerly the manager is called directly. Under ``torch.compile`` the
        calls go through the ``flextensor::pre_compute`` / ``post_compute``
        custom ops, which the compiler keeps in place around the unit's
        compute (custom_ops.py:267-328).

        The wrapper is bound to the module and runs the class's ``forward``
        on the module it is called on, so a copy of the model runs its own
        forward (the reason the reference patches with the unbound class
        function). A ``forward`` the caller had set on the instance is kept
        and put back by :meth:`release`.
        """
        module = unit.module
        own = module.__dict__.get("forward")
        mgr, label, mid = self, unit.label, id(self)

        def forward(self_module: nn.Module, *args: Any, **kwargs: Any) -> Any:
            def orig(*a: Any, **k: Any) -> Any:
                return own(*a, **k) if own is not None else type(self_module).forward(self_module, *a, **k)

            if (unit.compiled is not None and not torch.compiler.is_compiling() and not _COMPILED_CALL.active
                    and mgr.phase == OffloadPhase.INFERENCE):
                # Per-unit compiled graph: it re-enters this forward while tracing (the branch below).
                # Should the compiler run this frame eagerly instead, the flag sends the call down
                # the eager path rather than back into the compiled unit.
                _COMPILED_CALL.active = True
                try:
                    return unit.compiled(*args, **kwargs)
                finally:
                    _COMPILED_CALL.active = False
            if torch.compiler.is_compiling():
                if mgr.phase != OffloadPhase.INFERENCE:
                    raise RuntimeError(f"offload manager {mgr.name!r} is in {mgr.phase.value}: run the discovery and "
                                       "profiling passes eagerly, then compile")
                carrier = custom_ops.first_tensor((args, kwargs))
                if carrier is None:
                    raise RuntimeError(f"offload unit {label!r} has no tensor input to order its transfers against")
                torch.ops.flextensor.pre_compute(carrier, label, mid)
                out = orig(*args, **kwargs)
                produced = custom_ops.first_tensor(out)
                torch.ops.flextensor.post_compute(produced if produced is not None else carrier, label, mid)
                return out
            mgr._enter(label)
            try:
                return orig(*args, **kwargs)
            finally:
                mgr._exit(label)  # also when the unit raises, as the reference's trap exit does

        module.forward = types.MethodType(forward, module)
        self._patched.append((module, own))

    @staticmethod
    def _unpatch(patched: Sequence[tuple[nn.Module, Any]]) -> None:
        """Put back each module's own forward: the class's, or the one the caller had set on the instance."""
        for mod, own in patched:
            if own is not None:
                mod.forward = own
            elif "forward" in mod.__dict__:
                del mod.forward

    def _unit(self, label: str) -> _Unit:
        for u in self.units:
            if u.label == label:
                return u
        raise KeyError(label)

    def _enter(self, label: str) -> None:
        if self.phase == OffloadPhase.INFERENCE:
            if self._reload_pending and self.order and label == self.order[0]:
                self._reload_if_pending()  # a load on a submodule, which the root's load hook did not see
            if self._stale_encoding is not None:
                raise RuntimeError(f"offload manager {self.name!r}: {self._stale_encoding}")
            self.loader.enter(label)
            key = self._hbm_keys.get(label)
            if key is not None:
                self.controller.decode_resident(key)  # on the compute stream, ahead of the unit's kernels
            return
        if hip.is_capturing():
            raise RuntimeError(f"offload manager {self.name!r} is in {self.phase.value}: run the discovery and "
                               "profiling passes eagerly before capturing a graph")
        if label in self._seen_this_pass:
            raise NotImplementedError(f"offload unit {label!r} ran twice in one forward")
        u = self._unit(label)
        moved: list[nn.Parameter] = []
        try:
            for p in u.params:
                host = p.data
                p.data = host.to(self.device, non_blocking=False)
                self._cpu_data[id(p)] = host
                moved.append(p)
        except BaseException:
            # a move that failed part way (out of memory) puts back the ones already moved, so the host
            # originals are never overwritten by device copies on the next pass
            for p in moved:
                p.data = self._cpu_data.pop(id(p))
            raise
        self._seen_this_pass.append(label)
        if self.phase == OffloadPhase.PROFILING:
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            self._events[label] = (start, end)

    def _exit(self, label: str) -> None:
        if self.phase == OffloadPhase.INFERENCE:
            self.loader.exit(label)
            return
        if self.phase == OffloadPhase.PROFILING:
            self._events[label][1].record()
        u = self._unit(label)
        for p in u.params:
            p.data = self._cpu_data.pop(id(p))

    def _before_forward(self) -> None:
        """Bound the host's run-ahead: wait for the pass ``max_inflight_passes`` back.

        Under graph capture nothing is waited for: a captured pass is one
        fork/join region of the capturing stream, and replays are ordered by
        the stream they are launched on. A compiled forward skips this host
        bookkeeping (it must not enter the traced graph); its units' traps
        run as custom ops.
        """
        if torch.compiler.is_compiling():
            return
        if hip.is_capturing():
            if self.phase == OffloadPhase.INFERENCE and self.timing is not None and self.timing.enabled \
                    and not self.timing.graph_replay:
                raise RuntimeError("offload_timing='eager' cannot time a captured graph; "
                                   "capture with offload_timing='cuda_graph' or 'off'")
            return
        if self.phase in (OffloadPhase.DISCOVERY, OffloadPhase.PROFILING):
            # a pass that raised never reached the post-forward hook: drop what it left behind
            self._seen_this_pass = []
            self._events.clear()
        k = self.config.max_inflight_passes
        if self.phase == OffloadPhase.INFERENCE and k > 0 and len(self._pass_done) >= k:
            self._pass_done[-k].synchronize()

    def _after_forward(self) -> None:
        if torch.compiler.is_compiling():
            if self.phase != OffloadPhase.INFERENCE:
                raise RuntimeError(f"offload manager {self.name!r} is in {self.phase.value}: run the discovery and "
                                   "profiling passes eagerly, then compile")
            return
        if self.phase == OffloadPhase.INFERENCE:
            if hip.is_capturing():
                return
            if self.config.max_inflight_passes > 0:
                from .hip import HipEvent, current_stream

                self._pass_done.append(HipEvent().record(current_stream(self.device)))
                del self._pass_done[: -self.config.max_inflight_passes]
            self._advance_replan()
            return
        if self.phase == OffloadPhase.PROFILING and self._suspend_count:
            # a suspended profiling pass records no durations and does not use up profiling_iters
            self._events.clear()
            self._seen_this_pass = []
            return
        self._forwards += 1
        if self.phase == OffloadPhase.DISCOVERY:
            if not self.order:
                self.order = list(self._seen_this_pass)
            if self._forwards >= self._discovery_passes:
                self._finish_manual_discovery()
                self.phase = OffloadPhase.PROFILING
        elif self.phase == OffloadPhase.PROFILING:
            if not self.order:
                self.order = list(self._seen_this_pass)
            torch.cuda.synchronize(self.device)
            for label, (s, e) in self._events.items():
                self.durations.setdefault(label, []).append(s.elapsed_time(e))
            self._events.clear()
        self._seen_this_pass = []
        if self.phase == OffloadPhase.PROFILING and self._forwards >= self._discovery_passes + self.config.profiling_iters:
            self._to_inference()

    def _budget(self) -> int | None:
        """The plan's GPU byte budget (gpu_budget.py:66-113): ``max_gpu_mem_bytes``, else the fraction of
        the device's total memory, capped by what is available now.

        Available is the free memory plus the allocator's reusable cache, plus
        the tensors this manager already placed (the plan counts them, yet
        they no longer show as free). Less than 256 MiB available raises
        ``RuntimeError``.
        """
        cfg = self.config
        if cfg.max_gpu_mem_bytes is None and cfg.max_gpu_mem_fraction is None:
            return None
        free, total = torch.cuda.mem_get_info(self.device)
        cache = max(0, torch.cuda.memory_reserved(self.device) - torch.cuda.memory_allocated(self.device))
        if free + cache < MIN_GPU_BUDGET_BYTES:
            raise RuntimeError(f"Insufficient free GPU memory: {(free + cache) / 2**30:.2f} GiB available (free="
                               f"{free / 2**30:.2f}, reusable cache={cache / 2**30:.2f}), minimum required: "
                               f"{MIN_GPU_BUDGET_BYTES / 2**30:.2f} GiB")
        budget = cfg.max_gpu_mem_bytes if cfg.max_gpu_mem_bytes is not None else int(total * cfg.max_gpu_mem_fraction)
        available = free + cache + self._resident_bytes
        if budget > available:
            LOGGER.warning("offload %r: capping the GPU memory budget from %.2f GiB to %.2f GiB (%.2f GiB free, "
                           "%.2f GiB allocator cache, %.2f GiB already placed)", self.name, budget / 2**30,
                           available / 2**30, free / 2**30, cache / 2**30, self._resident_bytes / 2**30)
            budget = available
        return budget

    def _plan_from_state(self, state: TensorManagerState, budget: int | None = None,
                         encodable: Mapping[str, tuple[int, int]] | None = None) -> StreamPlan:
        for st in state.stats:
            if st.duration:
                self.durations.setdefault(st.label, []).append(st.duration)
        return plan_from_state(state, [self._unit(x) for x in self.order], self._resident_bytes,
                               self._budget() if budget is None else budget, encodable)

    def _encodable(self, units: Sequence[_Unit], budget: int | None) -> dict[str, tuple[int, int]] | None:
        """Per unit whose packed block encodes to under 0.9 of its bytes in the dense format (the one units
        kept in HBM use): (device bytes to reserve for the encoded block, bytes of the packed raw block). None when there is no budget or everything fits
        raw. The reservation adds max(64 KiB, 0.1% of the raw block) to the encoded size, room for a
        later state-dict load to re-encode in place."""
        if budget is None or self._resident_bytes + sum(u.nbytes for u in units) <= budget:
            return None
        from . import expcode
        from .layout import DEFAULT_ALIGNMENT

        t0 = time.perf_counter()
        out: dict[str, tuple[int, int]] = {}
        scratch: torch.Tensor | None = None
        for u in units:
            seen: set[int] = set()
            tensors = [p for p in u.params if not (id(p) in seen or seen.add(id(p)))]
            if not tensors or any(p.device.type != "cpu" for p in tensors):
                continue
            need = sum(p.numel() * p.element_size() for p in tensors) + DEFAULT_ALIGNMENT * len(tensors)
            if scratch is None or scratch.numel() < need:
                scratch = torch.empty(need, dtype=torch.uint8)
            size, raw = expcode.packed_encoded_size(tensors, DEFAULT_ALIGNMENT, scratch, dense=True)
            if raw == 0 or size > expcode.DEFAULT_MAX_RATIO * raw:
                continue
            reserve = (size + max(1 << 16, raw // 1024) + 255) // 256 * 256
            out[u.label] = (min(reserve, raw), raw)
        LOGGER.info("offload %r: encode_resident_blocks: %d of %d units encode below %.2f of their bytes "
                    "(sized in %.1f s)", self.name, len(out), len(units), expcode.DEFAULT_MAX_RATIO,
                    time.perf_counter() - t0)
        return out

    def _to_inference(self, state: TensorManagerState | None = None) -> None:
        t0 = time.perf_counter()
        cfg = self.config
        units_in_order = [self._unit(x) for x in self.order] if self.order else list(self.units)
        order = [u.label for u in units_in_order]
        blocks = max(cfg.num_blocks, 2)
        budget = self._budget()
        encodable = self._encodable(units_in_order, budget) if cfg.encode_resident_blocks else None
        if state is not None:
            self.plan = self._plan_from_state(state, budget, encodable)
        else:
            self.plan = plan_streaming(units_in_order, order, budget, self._resident_bytes, blocks,
                                       cfg.min_blocks, encodable)
        plan = self.plan
        self._validate_source_storage(plan)
        hbm = plan.encoded_resident
        resident_params = [p for x in plan.resident if x not in hbm for p in self._unit(x).params]
        with _oom_context(resident_params, f"the {len(plan.resident) - len(hbm)} offload units kept resident",
                          "Lower the budget (max_gpu_mem_fraction / max_gpu_mem_bytes) so that more units stream."):
            self._resident_bytes += self._upload_into(resident_params)
        layer_stats = [self._unit(x).stats(self._duration(x)) for x in order]
        if plan.block_data is None:
            self.loader = _ResidentLoader()
        else:
            bd = plan.block_data
            self._choose_copy_policy(plan, state)
            tensors_map = {id(p): p for x in [*plan.streamed, *hbm] for p in self._unit(x).params}
            pinner = self._pinner = HostPinner(cfg.pinned_memory_mode, enabled=cfg.pinned_memory)
            mode = nat.COPY_MODES[cfg.copy_engine]
            try:
                self._build_controller(cfg, plan, bd, tensors_map, pinner, mode, state)
            except (torch.cuda.OutOfMemoryError, nat.FtxOutOfMemoryError) as exc:
                host = sum(bd.label_to_size_map.values())
                slots = sum(bd.block_sizes.values())
                oom = torch.cuda.OutOfMemoryError(
                    f"out of memory while building the streaming blocks: {len(bd.label_to_size_map)} page-locked "
                    f"host blocks ({host / 2**30:.2f} GiB) and {len(bd.block_sizes)} GPU ring slots "
                    f"({slots / 2**30:.2f} GiB). The slots take GPU memory within the budget; the blocks take "
                    "page-locked host memory.")
                for key in ("_flextensor_cleanup_controller", "_flextensor_cleanup_error"):
                    if key in exc.__dict__:  # a retryable cleanup handle stays on the error the caller sees
                        oom.__dict__[key] = exc.__dict__[key]
                raise oom from exc
            bound = {tid: t.data for tid, t in tensors_map.items()}
            n_hooks = len(self._hooks)
            try:
                for tid, view in self.controller.get_tensor_id_to_view_mapping().items():
                    tensors_map[tid].data = view
                self._install_state_dict_hooks(tensors_map)
                reordered = plan.reordered if cfg.loader_order == "auto" else cfg.loader_order == "reordered"
                cls = (PreallocatedBatchTransferTensorLoaderReordered if reordered
                       else PreallocatedBatchTransferTensorLoader)
                self.timing = OffloadTimingCollector(order, enabled=cfg.offload_timing != "off",
                                                     graph_replay=cfg.offload_timing == "cuda_graph")
                policy = PiecewisePrefetchPolicy(enabled=cfg.piecewise_prefetch != "off",
                                                 strict=cfg.piecewise_prefetch == "error")
                # the loader's constructor preloads the first slots: the first copies run here
                self.loader = cls(layer_stats, self.device, bd.label_to_block_id, bd.transfer_to_compute_map,
                                  self.controller, self.timing, policy)
                self._apply_link_bound_order()
            except BaseException as primary:
                self._abort_build(primary, tensors_map, bound, n_hooks)
                raise
            self.controller.commit_construction()
        self.phase = OffloadPhase.INFERENCE
        if self.compile_fn is not None:
            raise_dynamo_limits(len(self.units))
            for u in self.units:
                if u.module is not None:  # manual blocks stay eager
                    u.compiled = self.compile_fn(u.module)
        self.build_seconds = time.perf_counter() - t0
        LOGGER.info("offload %r: %d streamed / %d resident units, %.1f s to build", self.name, len(plan.streamed),
                    len(plan.resident), self.build_seconds)
        if cfg.enable_diagnostics:
            LOGGER.info("offload %r plan:\n%s", self.name, self.plan_table())

    def _choose_copy_policy(self, plan: StreamPlan, state: TensorManagerState | None) -> None:
        """Choose the copy engine per chunk size from the measured host link (``FTX_COPY_AUTO``).

        At the INFERENCE transition the reference benchmarks the link live and
        plans with the curve (tensor_manager.py:1618-1630,
        memory_transfer_benchmark.py:59-129). Here both copy engines are timed
        at sizes up to the largest streamed unit; the zero-copy kernel takes
        the chunk sizes where it is at least 10% faster than SDMA
        (:func:`~flextensor_amd.link_model.choose_copy_policy`), and the SDMA
        curve becomes ``memory_transfer_stats``. A plan restored from a saved
        state reapplies the saved policy without measuring, as the reference
        rebuilds its curve from the saved statistics. Only ``copy_engine="auto"``
        consults the policy; ``link_benchmark=False`` keeps the library default.

        The policy belongs to this manager: its controller passes it with
        every copy (``ftx_copy_h2d_policy``), and nothing in the library's
        process-wide state changes, so named managers streaming side by side
        each copy under their own measurement, as the reference's named
        managers copy independently (offload_manager.py:2817-2850).

        A measured policy then looks at the pass: when the profiled compute of
        its units is under 0.4 of the curve's time for its streamed units
        (:func:`~flextensor_amd.link_model.is_link_bound`), every ring copy
        goes to the zero-copy kernel at a small grid, which removes the idle
        gap between consecutive SDMA copies. A pass with no profiled durations
        keeps the measured policy.
        """
        cfg = self.config
        link = None
        if state is not None and state.copy_policy:
            link = LinkMeasurement.from_dict(state.copy_policy, source="profile")
        elif cfg.link_benchmark and cfg.copy_engine == "auto" and plan.streamed:
            largest = max(self._unit(x).nbytes for x in plan.streamed)
            try:
                link = measure_link(link_probe_sizes(largest), self.device)
            except (nat.FtxError, RuntimeError) as exc:  # an optimisation only: stream with the default policy
                LOGGER.warning("offload %r: measuring the host link failed (%s); keeping the default copy policy",
                               self.name, exc)
                torch.cuda.empty_cache()
        if link is None:
            return
        if link.source == "measured" and any(self.durations.get(x) for x in plan.streamed):
            compute_ms = sum(self._duration(x) for x in [*plan.streamed, *plan.resident])
            sizes = [self._unit(x).nbytes for x in plan.streamed]
            transfer_ms = link.transfer_ms(sizes)
            link = dataclasses.replace(link, pass_compute_ms=compute_ms, pass_transfer_ms=transfer_ms)
            if is_link_bound(compute_ms, transfer_ms):
                link = link.for_link_bound_pass(max(sizes))
        self.link = link
        self.memory_transfer_stats = link.memory_transfer_stats()
        LOGGER.info("offload %r: %s", self.name, link.describe())

    def _measured_compute_bound(self) -> bool:
        """The link measurement profiled this pass and found its compute too long for encoded transfers
        to pay: 0.9 of its raw transfer time or more (:func:`~flextensor_amd.link_model.encoding_pays`)."""
        link = self.link
        if link is None or link.pass_compute_ms is None or link.pass_transfer_ms is None:
            return False
        return not encoding_pays(link.pass_compute_ms, link.pass_transfer_ms)

    def _apply_link_bound_order(self) -> None:
        """A link-bound pass orders its ring waits for the link; any other pass keeps the reference's order.

        While the compute stream waits on a copy's ready event, that copy
        loses 35-40 us per 386 MiB on the MI355X (0.5% of its rate). In a
        link-bound pass the compute stream has nothing to run meanwhile, so
        the reordered loader blocks the host on the copy instead, with the
        next copy already queued; the default loader (every unit streamed)
        releases the slots a unit read before it waits for the next copy,
        so the copy after that queues behind it (``link_bound``). A
        compute-bound pass keeps the reference's order and stream waits,
        which let the host run ahead.
        """
        if hasattr(self.loader, "link_bound"):
            self.loader.link_bound = bool(self.link is not None and self.link.link_bound)
        # Encoded blocks (encode_streamed_blocks) carry fewer bytes, and their decode holds 16 CUs while it
        # runs: worth it until the pass's compute reaches 0.9 of its raw transfer time.
        if getattr(self.controller, "encoded", None):
            self.controller.use_encoded = not self._measured_compute_bound()

    def _abort_build(self, primary: BaseException, tensors_map: dict[int, torch.Tensor],
                     bound: dict[int, torch.Tensor], n_hooks: int) -> None:
        """Undo a streaming build that failed after its controller was made (tensor_manager.py:1585-1596).

        Parameters go back to what they held before they were bound to slot
        views, the state-dict hooks of the build go, and the controller's
        ``abort_construction`` restores the released sources and frees the
        host blocks, the GPU slots and any shared-memory segments. A cleanup
        that fails never replaces ``primary``: the controller stays reachable
        from it (``_flextensor_cleanup_controller``) so ``shutdown()`` can be
        retried. Copies the loader already queued are waited for first, since
        they read the host blocks about to be freed.
        """
        try:
            torch.cuda.synchronize(self.device)
        except Exception:  # noqa: BLE001 - the device may be what failed; the primary error is the one to report
            LOGGER.warning("offload %r: synchronize before undoing the build failed", self.name, exc_info=True)
        for h in self._hooks[n_hooks:]:
            h.remove()
        del self._hooks[n_hooks:]
        for tid, t in tensors_map.items():
            t.data = bound[tid]
        self.loader = self.timing = None
        self._hbm_keys, self._stale_encoding = {}, None
        controller, self.controller = self.controller, None
        if controller is not None:
            controller.abort_construction(primary)
        self._release_pins()

    def _validate_source_storage(self, plan: StreamPlan) -> None:
        """Refuse streamed tensors that overlap another distinct tensor's bytes, before anything moves.

        Each tensor is packed into its block on its own, so two views of the
        same bytes would stop aliasing once streamed (loaders.py:1217-1243).
        Disjoint views of one storage (parameters that view a released host
        block) are fine.
        """
        managed = [p for x in plan.streamed for p in self._unit(x).params]
        if not managed or self.model is None:
            return
        others = [t for _, t in self.model.named_parameters(remove_duplicate=False)]
        others += [t for _, t in self.model.named_buffers(remove_duplicate=False) if t is not None]
        groups = overlapping_views(managed, others)
        if groups:
            names: dict[int, str] = {}
            for n, t in list(self.model.named_parameters(remove_duplicate=False)) + list(
                    self.model.named_buffers(remove_duplicate=False)):
                names.setdefault(id(t), n)
            shown = [sorted(names.get(i, f"tensor id {i}") for i in g) for g in groups]
            raise ValueError("Block loaders cannot preserve distinct tensor views sharing storage with overlapping "
                             f"byte regions ({shown}); give them separate storage (clone one) or keep their "
                             "modules out of the offload units")

    def _install_state_dict_hooks(self, streamed: dict[int, torch.Tensor]) -> None:
        """Serialize streamed parameters from their host blocks, and load into them.

        While streaming, a streamed parameter views a ring slot that holds
        whichever unit was loaded last, so ``state_dict()`` takes such a
        parameter's bytes from its host block (the authoritative copy, viewed
        without a copy, as a state dict views parameters). ``load_state_dict()``
        writes them there too: for the load the parameter points at its host
        block, so no slot is written (a slot write would also race the
        transfers filling the ring). ``assign=True`` would replace the aliased
        parameters and is refused; ``keep_vars=True`` keeps the live parameters.
        """
        assert self.model is not None and self.controller is not None
        host: dict[int, torch.Tensor] = {}
        for label in self.controller.block_map_cpu:
            for tid, view in zip(self.controller.label_to_cpu_tensor_id_map[label], self._cpu_views(label)):
                host[tid] = view
        owners: dict[int, tuple[nn.Module, dict[str, nn.Parameter]]] = {}
        for mod in self.model.modules():
            for key, p in mod._parameters.items():
                if p is not None and id(p) in host and id(p) in streamed:
                    owners.setdefault(id(mod), (mod, {}))[1][key] = p
        name, device, mgr = self.name, self.device, self
        streamed_view = {tid: t.data for tid, t in streamed.items()}

        for mod, local in owners.values():
            def save_hook(module: nn.Module, state_dict: dict, prefix: str, _meta: Any,
                          local: dict[str, nn.Parameter] = local) -> None:
                for key, p in local.items():
                    k = prefix + key
                    if k in state_dict and not isinstance(state_dict[k], nn.Parameter):
                        state_dict[k] = host[id(p)]

            def before_load(module: nn.Module, *_args: Any, local: dict[str, nn.Parameter] = local,
                            **_kwargs: Any) -> None:
                torch.cuda.synchronize(device)  # no transfer may still be reading a host block
                for p in local.values():
                    p.data = host[id(p)]

            def after_load(module: nn.Module, _incompatible: Any, local: dict[str, nn.Parameter] = local) -> None:
                mgr._reload_pending = True
                for key, p in local.items():
                    p.data = streamed_view[id(p)]
                    if module._parameters.get(key) is not p:
                        raise RuntimeError(f"offload manager {name!r}: load_state_dict(assign=True) replaced the "
                                           f"streamed parameter {key!r}; release() the model before assigning")

            self._hooks.append(mod.register_state_dict_post_hook(save_hook))
            self._hooks.append(mod._register_load_state_dict_pre_hook(before_load, with_module=True))
            self._hooks.append(mod.register_load_state_dict_post_hook(after_load))
        # The root's load hook runs after every submodule's: reload the next pass's first slots, which the
        # previous pass already filled from the old bytes.
        self._hooks.append(self.model.register_load_state_dict_post_hook(lambda *_: mgr._reload_if_pending()))

    def _reload_if_pending(self) -> None:
        """After new streamed bytes were loaded, refill the slots the previous pass preloaded."""
        if not self._reload_pending or self.phase != OffloadPhase.INFERENCE or hip.is_capturing():
            return
        self._reload_pending = False
        # the new host bytes reach the link, or the units kept encoded in HBM, only once re-encoded
        if getattr(self.controller, "encoded", None) or getattr(self.controller, "hbm_encoded", None):
            torch.cuda.synchronize(self.device)
            try:
                self.controller.refresh_encoded()
            except ValueError as exc:
                # Every later forward raises: the encoded blocks would feed the old weights. A graph captured
                # before the load must not be replayed either.
                self._stale_encoding = f"{exc} (the encoded blocks no longer hold the loaded weights)"
                raise
        preload = getattr(self.loader, "preload", None)
        if preload is not None:
            preload()

    def _build_controller(self, cfg: OffloadConfig, plan: StreamPlan, bd: Any, tensors_map: dict[int, torch.Tensor],
                          pinner: HostPinner, mode: int, state: TensorManagerState | None) -> None:
        """The block controller of the plan: packed host blocks and GPU ring slots, copying under this
        manager's copy policy (the library default when no link was measured or restored)."""
        policy = self.link.native_policy() if self.link is not None else None
        if cfg.transfer_mode == "raw_block_transfer":
            self.controller = RawBlockController(bd.label_to_size_map, bd.block_sizes, self.device, tensors_map,
                                                 plan.strategy_map, bd.label_to_block_id, host_pinner=pinner,
                                                 copy_mode=mode, copy_policy=policy)
        else:
            shm_names: dict[str, str] | None = None
            if cfg.shm_enabled:
                if self._load_from_shm:
                    assert state is not None and state.shm_block_name_map
                    shm_names = dict(state.shm_block_name_map)
                else:
                    labels = [x for group in bd.allocation_ordered.values() for x in group
                              if plan.strategy_map.get(x)]
                    shm_names = {x: f"{cfg.shm_namespace}_b{i}" for i, x in enumerate(labels)}
            # Units kept encoded in HBM: one more slot group, keyed apart from the ring's transfer labels
            allocation_ordered, strategy_map, l2b = bd.allocation_ordered, plan.strategy_map, bd.label_to_block_id
            keys = {x: f"hbm::{x}" for x in plan.encoded_resident}
            if keys:
                clash = set(keys.values()) & set(strategy_map)
                if clash:
                    raise ValueError(f"offload unit labels {sorted(clash)} clash with the keys of units kept "
                                     "encoded in HBM; rename them or turn encode_resident_blocks off")
                tier = min(allocation_ordered, default=0) - 1
                allocation_ordered = {**allocation_ordered, tier: list(keys.values())}
                strategy_map = {**strategy_map, **{k: list(self._unit(x).stats().tensors) for x, k in keys.items()}}
                l2b = {**l2b, **{k: tier for k in keys.values()}}
            self.controller = AllocationBlockController(allocation_ordered, self.device, tensors_map,
                                                        strategy_map, l2b,
                                                        host_pinner=pinner, copy_mode=mode, copy_policy=policy,
                                                        shm_block_name_map=shm_names,
                                                        load_from_shm=self._load_from_shm,
                                                        encode_blocks=cfg.encode_streamed_blocks
                                                        and not self._measured_compute_bound(),
                                                        hbm_encoded={keys[x]: n
                                                                     for x, n in plan.encoded_resident.items()})
            self._hbm_keys = keys
            if cfg.encode_streamed_blocks and not self.controller.encoded:
                LOGGER.info("offload %r: encode_streamed_blocks: %s; the blocks cross the link raw", self.name,
                            "the pass is compute-bound" if self._measured_compute_bound()
                            else "no streamed block shrinks by a tenth")

    def plan_table(self) -> str:
        """Per unit: bytes, profiled ms, and where it lives (its slot and transfer label when streamed)."""
        plan = self.plan
        if plan is None:
            return "(no plan yet)"
        bd = plan.block_data
        producer = {c: t for t, c in bd.transfer_to_compute_map.items()} if bd else {}
        rows = [f"{'unit':<32} {'MB':>10} {'ms':>9}  placement"]
        for label in self.order:
            u = self._unit(label)
            if label in plan.streamed and bd is not None:
                src = producer.get(label, "?")
                where = f"slot {bd.label_to_block_id.get(src, '?')}, loaded during {src!r}"
            elif label in plan.encoded_resident:
                where = f"resident, exponent-coded in HBM ({plan.encoded_resident[label] / 2**20:.2f} MB)"
            else:
                where = "resident"
            rows.append(f"{label:<32} {u.nbytes / 2**20:>10.2f} {self._duration(label):>9.3f}  {where}")
        if self.link is not None:
            rows.append(self.link.describe())
            rows.append(format_memory_transfer_table(self.link.memory_transfer_stats()))
        probe = hip.transfer_stream_probe(self.device) if self.device is not None else None
        if probe is not None:
            rows.append(f"transfer stream: candidate {probe['chosen_candidate']} of {probe['attempts']} "
                        f"({probe['rejected']} rejected for queueing behind the compute stream)")
        return "\n".join(rows)


class _ResidentLoader:
    """Everything fits the budget: traps do nothing."""

    def enter(self, label: str) -> None:
        return None

    def exit(self, label: str) -> None:
        return None

    def shutdown(self) -> None:
        return None

    def get_gpu_memory_bytes(self) -> int:
        return 0


class _DiscoveryMode(TorchFunctionMode):
    """Sees every torch call while manual blocks are discovered; places the parameters it is handed."""

    def __init__(self, mgr: OffloadManager) -> None:
        super().__init__()
        self.mgr = mgr

    def __torch_function__(self, func: Any, types: Any, args: Any = (), kwargs: Any = None) -> Any:
        kwargs = kwargs or {}
        pending = self.mgr._pending
        if pending and not self.mgr._quiet:
            for t in tree_leaves((args, kwargs)):
                if isinstance(t, torch.Tensor) and id(t) in pending and pending[id(t)] is t:
                    self.mgr._touch(t)
        return func(*args, **kwargs)


class OffloadBlock:
    """``with manager.offload_block(label):`` (the trap the reference returns, trap_tensor_mode.py:376-397)."""

    def __init__(self, mgr: OffloadManager, label: str) -> None:
        self.manager = mgr
        self.label = label
        self._kind: str | None = None

    def __enter__(self) -> OffloadBlock:
        self._kind = self.manager._block_enter(self.label)
        return self

    def __exit__(self, *exc: Any) -> None:
        kind, self._kind = self._kind, None
        if kind is not None:
            self.manager._block_exit(self.label, kind)


_MANAGERS: dict[str, OffloadManager] = {}
_MANAGERS_LOCK = threading.Lock()


def get_offload_manager(name: str = DEFAULT_MANAGER_NAME) -> OffloadManager:
    """The manager registered under ``name``, created on first use by the calling thread
    (offload_manager.py:2815-2850); another thread's manager raises ``RuntimeError``."""
    with _MANAGERS_LOCK:
        mgr = _MANAGERS.get(name)
        if mgr is None:
            mgr = _MANAGERS[name] = OffloadManager(name)
    mgr._check_thread()
    return mgr


def offload(model: nn.Module, config: OffloadConfig | None = None, name: str = DEFAULT_MANAGER_NAME,
            compile_fn: Callable[[nn.Module], Any] | None = None) -> nn.Module:
    """Patch ``model`` so its offload units stream from pinned host memory.

    ``compile_fn`` compiles each offload unit separately once streaming starts
    (offload_manager.py:2858-2884).
    """
    return get_offload_manager(name).offload(model, config, compile_fn=compile_fn)


def init(config: OffloadConfig | None = None, name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).init(config)


def set_config(config: OffloadConfig, name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).set_config(config)


def offload_units(name: str = DEFAULT_MANAGER_NAME) -> tuple[tuple[str, nn.Module], ...]:
    return get_offload_manager(name).offload_units()


def resident_units(name: str = DEFAULT_MANAGER_NAME) -> tuple[tuple[str, nn.Module], ...]:
    return get_offload_manager(name).resident_units()


def clear_profiling_durations(name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).clear_profiling_durations()


def suspend_profiling(name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).suspend_profiling()


def resume_profiling(name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).resume_profiling()


@contextlib.contextmanager
def pause_profiling(name: str = DEFAULT_MANAGER_NAME) -> Iterator[None]:
    with get_offload_manager(name).pause_profiling():
        yield


def request_strategy_replan(name: str = DEFAULT_MANAGER_NAME, *, manual_update_state: bool = False) -> int:
    """:meth:`OffloadManager.request_strategy_replan` of the named manager (offload_manager.py:3091-3107)."""
    return get_offload_manager(name).request_strategy_replan(manual_update_state=manual_update_state)


def update_state(name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).update_state()


def update_offload_timing(name: str = DEFAULT_MANAGER_NAME) -> bool:
    return get_offload_manager(name).update_offload_timing()


def offload_block(block_name: str, name: str = DEFAULT_MANAGER_NAME) -> OffloadBlock:
    """Manual offload block of the named manager (offload_manager.py:2990-2998)."""
    return get_offload_manager(name).offload_block(block_name)


def release(name: str = DEFAULT_MANAGER_NAME, preserve_model: bool = True) -> None:
    mgr = _MANAGERS.pop(name, None)
    if mgr is not None:
        mgr.release(preserve_model)


def get_gpu_memory_usage(name: str = DEFAULT_MANAGER_NAME) -> GPUMemoryUsage:
    return get_offload_manager(name).get_gpu_memory_usage()


def collect_offload_timing(name: str = DEFAULT_MANAGER_NAME) -> OffloadTimingReport | None:
    return get_offload_manager(name).collect_offload_timing()


def reset_offload_timing(name: str = DEFAULT_MANAGER_NAME) -> None:
    get_offload_manager(name).reset_offload_timing()


def save_profile(profile_directory: str | None = None, name: str = DEFAULT_MANAGER_NAME) -> str:
    """Save the named manager's plan as ``<dir>/profile.json`` (offload_manager.py:2898-2907)."""
    return get_offload_manager(name).save_profile(profile_directory)


def load_profile(profile_directory: str | None = None, model: nn.Module | None = None,
                 name: str = DEFAULT_MANAGER_NAME) -> None:
    """Adopt a saved profile in the named manager (offload_manager.py:2910-2922)."""
    get_offload_manager(name).load_profile(profile_directory, model)


def offload_from_profile(model: nn.Module, profile_directory: str | os.PathLike[str] | None,
                         config: OffloadConfig | None = None, name: str = DEFAULT_MANAGER_NAME,
                         compile_fn: Callable[[nn.Module], Any] | None = None) -> nn.Module:
    """Offload ``model`` straight into streaming with a saved plan: no discovery or profiling passes.

    Same signature as the reference (offload_manager.py:2961-2986); ``profile_directory`` None
    falls back to ``config.profile_storage_dir``.
    """
    if isinstance(profile_directory, OffloadConfig):
        raise TypeError("offload_from_profile(model, profile_directory, config=...): the second argument is the "
                        "profile directory")
    cfg = config or OffloadConfig()
    directory = profile_directory or cfg.profile_storage_dir
    if directory is None:
        raise ValueError("No profile directory specified. Provide profile_directory argument "
                         "or set profile_storage_dir in OffloadConfig.")
    return get_offload_manager(name).offload(model, cfg, state=load_state(os.fspath(directory)),
                                             compile_fn=compile_fn)


def offload_from_state(model: nn.Module, state: TensorManagerState, config: OffloadConfig | None = None,
                       name: str = DEFAULT_MANAGER_NAME) -> nn.Module:
    """Adopt an in-memory saved plan (offload_manager.py:2925-2958); ``state`` must use ``config``'s transfer mode."""
    mgr = get_offload_manager(name)
    return mgr.offload_from_state(model, state, config or mgr.config or OffloadConfig())
