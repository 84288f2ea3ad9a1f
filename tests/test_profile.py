"""Saved profiles (schema 3): JSON shape, consistency checks, plan round trip.

The fixtures marked with a reference location are transcribed from the
reference's own tests; the round trip checks that a plan written by
:func:`state_from_plan` and read back by :func:`plan_from_state` gives the
same slot plan, streamed set and loader order as the planner produced.
"""

from __future__ import annotations

import json
import struct

import pytest
import torch

from flextensor_amd import workloads as W
from flextensor_amd.manager import (
    _Unit,
    plan_from_state,
    plan_streaming,
    select_offload_units,
    state_from_plan,
)
from flextensor_amd.planner import LayerStatistics, TensorStatistics, check_overlap_constraint
from flextensor_amd.profile import (
    PROFILE_FILE,
    TensorManagerState,
    load_state,
    load_state_from_bytes,
    save_state,
    save_state_to_bytes,
)


def _mock_state(names: list[str], view_names: list[str] | None = None) -> TensorManagerState:
    """The shape of tests/unit/test_state_handler_validation.py:58-96 (strategy loader, one label)."""
    view_names = view_names or []
    inventory = [*names, *(n for n in view_names if n not in names)]
    ids = {n: i for i, n in enumerate(inventory)}

    def ts():
        return [TensorStatistics(i, n, 1000, 0.1) for i, n in enumerate(names)]

    return TensorManagerState(
        loader_type="strategy",
        tensor_id_to_name_map=dict(enumerate(inventory)),
        allocation_ordered={},
        label_to_size_map={},
        block_sizes={},
        load_strategy={"layer_0": ts()},
        release_strategy={"layer_0": ts()},
        label_to_block_id={},
        stats=[LayerStatistics("layer_0", ts(), 1.0)],
        transfer_to_compute_map={},
        view_tensors_ids=[ids[n] for n in view_names],
        view_tensors_names=view_names,
        gpu_tensors_names=[],
        shm_block_name_map=None,
    )


# ---- fixtures from the reference's tests --------------------------------------


def test_reference_duplicate_inventory_names_rejected():
    # tests/unit/test_state_handler_validation.py:99-104
    data = _mock_state(["first", "second"]).to_dict()
    data["tensor_id_to_name_map"]["1"] = "first"
    with pytest.raises(ValueError, match=r"inventory names.*unique"):
        TensorManagerState.from_dict(data)


def test_reference_unknown_loader_type_rejected():
    # tests/unit/test_state_handler_validation.py:107-112
    data = _mock_state(["weight"]).to_dict()
    data["loader_type"] = "unknown"
    with pytest.raises(ValueError, match="Unknown loader type"):
        TensorManagerState.from_dict(data)


def test_reference_statistic_identity_mismatch_rejected():
    # tests/unit/test_state_handler_validation.py:115-120
    data = _mock_state(["weight"]).to_dict()
    data["load_strategy"]["layer_0"][0]["tensor_id"] = -1
    with pytest.raises(ValueError, match=r"TensorStatistics.*tensor_id.*name"):
        TensorManagerState.from_dict(data)


def test_reference_profile_file_loads(tmp_path):
    # tests/unit/test_offload_manager_profile.py:428-471: a minimal strategy profile on disk
    d = tmp_path / "profile"
    d.mkdir()
    (d / PROFILE_FILE).write_text(json.dumps({
        "version": TensorManagerState.SCHEMA_VERSION,
        "loader_type": "strategy",
        "tensor_id_to_name_map": {"123": "layer.weight"},
        "allocation_ordered": {},
        "label_to_size_map": {},
        "block_sizes": {},
        "load_strategy": {},
        "release_strategy": {},
        "label_to_block_id": {},
        "stats": [],
        "transfer_to_compute_map": {},
        "view_tensors_ids": [123],
        "view_tensors_names": ["layer.weight"],
        "gpu_tensors_names": [],
        "shm_block_name_map": None,
    }))
    st = load_state(d)
    assert st.loader_type == "strategy"
    assert st.tensor_id_to_name_map == {123: "layer.weight"}
    assert st.view_tensors_ids == [123]


def test_reference_missing_profile_raises(tmp_path):
    # tests/unit/test_offload_manager_profile.py:473-485
    with pytest.raises(FileNotFoundError):
        load_state(tmp_path / "nonexistent")


# ---- schema version -------------------------------------------------------------


@pytest.mark.parametrize("version,match", [(4, "newer than supported"), (2, "outdated"), (None, "outdated")])
def test_schema_version_checked(version, match):
    data = _mock_state(["w"]).to_dict()
    if version is None:
        del data["version"]  # a file with no version is version 1
    else:
        data["version"] = version
    with pytest.raises(ValueError, match=match):
        TensorManagerState.from_dict(data)


def test_non_object_json_rejected(tmp_path):
    (tmp_path / PROFILE_FILE).write_text("[1, 2]")
    with pytest.raises(ValueError, match="JSON object"):
        load_state(tmp_path)


# ---- managed tensor metadata (tests/unit/test_state_handler_shm.py) ------------------------


def _block_state() -> TensorManagerState:
    """tests/unit/test_state_handler_shm.py:16-44: an allocation-block plan of two labels."""
    ts = [TensorStatistics(0, "layer0.weight", 1024, 0.1), TensorStatistics(1, "layer1.weight", 2048, 0.2),
          TensorStatistics(2, "layer2.weight", 512, 0.05)]
    return TensorManagerState(
        loader_type="allocation_block_transfer",
        tensor_id_to_name_map={0: "layer0.weight", 1: "layer1.weight", 2: "layer2.weight"},
        allocation_ordered={0: ["trap_0"], 1: ["trap_1"]},
        label_to_size_map={"trap_0": 3072, "trap_1": 512},
        block_sizes={0: 3072, 1: 512},
        load_strategy={"trap_0": ts[:2], "trap_1": ts[2:]},
        release_strategy={"trap_0": ts[:2], "trap_1": ts[2:]},
        label_to_block_id={"trap_0": 0, "trap_1": 1},
        stats=[LayerStatistics("trap_0", ts[:2], 1.0), LayerStatistics("trap_1", ts[2:], 0.5)],
        transfer_to_compute_map={"trap_0": "trap_0", "trap_1": "trap_1"},
        view_tensors_ids=[0, 1, 2],
        view_tensors_names=["layer0.weight", "layer1.weight", "layer2.weight"],
        gpu_tensors_names=[],
        shm_block_name_map=None,
    )


def test_block_state_round_trips_and_legacy_metadata_loads():
    data = _block_state().to_dict()
    assert data["version"] == 3 and TensorManagerState.from_dict(data).to_dict() == data
    data.pop("managed_tensor_dtypes")
    data.pop("managed_tensor_layouts")
    legacy = TensorManagerState.from_dict(data)
    assert legacy.managed_tensor_dtypes == {} and legacy.managed_tensor_layouts == {}


@pytest.mark.parametrize("first_layout", [{"shape": [16, 16], "stride": [1, 16]}, {"shape": [16, 16], "stride": [16, 1]},
                                          {"shape": [1, 256], "stride": [0, 1]},
                                          {"shape": [4, 4, 16], "stride": [4, 1, 16]}])
def test_mixed_dtypes_and_packed_layouts_round_trip_through_bytes(first_layout):
    st = _block_state()
    st.managed_tensor_dtypes = {"layer0.weight": "float32", "layer1.weight": "bfloat16",
                                "layer2.weight": "float8_e4m3fn"}
    st.managed_tensor_layouts = {"layer0.weight": first_layout, "layer1.weight": {"shape": [32, 32], "stride": [32, 1]},
                                 "layer2.weight": {"shape": [512], "stride": [1]}}
    back = load_state_from_bytes(save_state_to_bytes(st))
    assert back.managed_tensor_dtypes == st.managed_tensor_dtypes
    assert back.managed_tensor_layouts == st.managed_tensor_layouts


@pytest.mark.parametrize("table,entry", [("managed_tensor_layouts", {"shape": [256], "stride": [1]}),
                                         ("managed_tensor_dtypes", "float32")])
def test_metadata_must_cover_every_managed_tensor(table, entry):
    data = _block_state().to_dict()
    data[table] = {"layer0.weight": entry}
    with pytest.raises(ValueError, match=table + r".*cover every managed tensor"):
        TensorManagerState.from_dict(data)


@pytest.mark.parametrize("layout", [{"shape": [256]}, {"shape": [16, 16], "stride": [1]}, {"shape": [-256], "stride": [1]},
                                    {"shape": [256], "stride": [-1]}, {"shape": [256], "stride": [2]},
                                    {"shape": [256], "stride": [0]}, {"shape": [True], "stride": [1]},
                                    {"shape": [256], "stride": [True]}, {"shape": [3, 3], "stride": [2, 2]},
                                    {"shape": [1, 256], "stride": [2**64, 1]}])
def test_layouts_that_are_not_packed_are_rejected(layout):
    """Gaps, overlaps, negative or boolean values, rank mismatches and strides past int64 (:105-127)."""
    data = _block_state().to_dict()
    data["managed_tensor_layouts"] = {"layer0.weight": layout, "layer1.weight": {"shape": [512], "stride": [1]},
                                      "layer2.weight": {"shape": [128], "stride": [1]}}
    with pytest.raises(ValueError, match="invalid layout metadata"):
        TensorManagerState.from_dict(data)


@pytest.mark.parametrize("dtype_name", ["not_a_torch_dtype", "Tensor", "", "float"])
def test_dtype_names_must_be_canonical_torch_dtypes(dtype_name):
    data = _block_state().to_dict()
    data["managed_tensor_dtypes"] = {"layer0.weight": "float32", "layer1.weight": dtype_name,
                                     "layer2.weight": "float32"}
    with pytest.raises(ValueError, match=r"invalid dtype metadata for 'layer1.weight'"):
        TensorManagerState.from_dict(data)


def test_state_loads_from_a_shared_memory_buffer():
    """:169-183: the bytes form read back out of a POSIX shared-memory segment."""
    from multiprocessing.shared_memory import SharedMemory

    st = _block_state()
    blob = save_state_to_bytes(st)
    shm = SharedMemory(create=True, size=len(blob) + 1024)
    try:
        shm.buf[:len(blob)] = blob
        back = load_state_from_bytes(bytes(shm.buf[:len(blob)]))
        assert back.allocation_ordered == st.allocation_ordered and back.label_to_block_id == st.label_to_block_id
        assert [(t.name, t.size_bytes) for t in back.load_strategy["trap_0"]] == \
            [(t.name, t.size_bytes) for t in st.load_strategy["trap_0"]]
        assert [(x.label, x.duration) for x in back.stats] == [(x.label, x.duration) for x in st.stats]
    finally:
        shm.close()
        shm.unlink()


def test_short_buffers_name_what_is_missing():
    with pytest.raises(ValueError, match=r"Buffer too short.*length prefix"):
        load_state_from_bytes(b"")
    with pytest.raises(ValueError, match=r"Buffer too short.*1000 bytes"):
        load_state_from_bytes(struct.pack("!I", 1000) + b"x" * 10)


# ---- bytes form -------------------------------------------------------------------


def test_bytes_round_trip_and_prefix():
    st = _mock_state(["a", "b"], ["a"])
    blob = save_state_to_bytes(st)
    n = int.from_bytes(blob[:4], "big")
    assert n == len(blob) - 4
    assert json.loads(blob[4:])["version"] == 3
    assert load_state_from_bytes(blob).to_dict() == st.to_dict()
    assert load_state_from_bytes(memoryview(blob + b"trailing")).to_dict() == st.to_dict()
    with pytest.raises(ValueError, match="too short"):
        load_state_from_bytes(blob[:3])
    with pytest.raises(ValueError, match="too short"):
        load_state_from_bytes(blob[:-1])


# ---- plan -> state -> JSON -> state -> plan ----------------------------------------


def _units(model):
    name_of = {id(p): n for n, p in model.named_parameters()}
    labels = select_offload_units(model, ["layers.*"], [])
    seen: set[int] = set()
    out = []
    for label in labels:
        mod = model.get_submodule(label)
        params = [p for p in mod.parameters() if id(p) not in seen]
        seen.update(id(p) for p in params)
        out.append(_Unit(label, mod, params, [name_of[id(p)] for p in params]))
    return out


@pytest.mark.parametrize("budget_layers", [None, 5, 7])
@pytest.mark.parametrize("loader_type", ["allocation_block_transfer", "raw_block_transfer"])
def test_plan_state_round_trip(tmp_path, budget_layers, loader_type):
    model = W.build_mlp_stack(10, 64, 176, seed=3)
    units = _units(model)
    order = [u.label for u in units]
    layer = units[0].nbytes
    budget = None if budget_layers is None else budget_layers * layer
    plan = plan_streaming(units, order, budget, 0, 2)
    durations = {x: 1e-3 * (i + 1) for i, x in enumerate(order)}
    st = state_from_plan(model, units, plan, durations, loader_type)
    st.validate_internal()
    save_state(st, tmp_path)
    assert not [p for p in tmp_path.iterdir() if p.name != PROFILE_FILE]  # no temporary file left behind
    back = load_state(tmp_path)
    assert back.to_dict() == st.to_dict()

    # a fresh model of the same architecture: new tensor ids, same names
    twin = W.build_mlp_stack(10, 64, 176, seed=3)
    twin_units = _units(twin)
    again = plan_from_state(back, twin_units, 0, budget)
    assert again.streamed == plan.streamed and again.resident == plan.resident
    assert again.reordered == plan.reordered
    if plan.block_data is None:
        assert again.block_data is None
    else:
        assert again.block_data == plan.block_data
        assert again.planned_gpu_bytes == plan.planned_gpu_bytes
        twin_ids = {id(p) for p in twin.parameters()}
        names = {k: [t.name for t in v] for k, v in plan.strategy_map.items()}
        assert {k: [t.name for t in v] for k, v in again.strategy_map.items()} == names
        assert all(t.tensor_id in twin_ids for v in again.strategy_map.values() for t in v)
        stats = [u.stats() for u in twin_units]
        assert check_overlap_constraint(again.block_data.transfer_to_compute_map, stats,
                                        again.block_data.label_to_block_id)
    assert [s.duration for s in back.stats] == [durations[x] for x in order]
    assert set(back.gpu_tensors_names) | set(back.view_tensors_names) == {n for n, _ in model.named_parameters()}


def test_plan_from_state_rejects_changed_model(tmp_path):
    model = W.build_mlp_stack(6, 64, 176, seed=0)
    units = _units(model)
    plan = plan_streaming(units, [u.label for u in units], None, 0, 2)
    st = state_from_plan(model, units, plan, {}, "allocation_block_transfer")
    wider = W.build_mlp_stack(6, 64, 192, seed=0)
    with pytest.raises(ValueError, match="different size"):
        plan_from_state(st, _units(wider), 0, None)
    as_f32 = W.build_mlp_stack(6, 64, 176, seed=0).float()
    with pytest.raises(ValueError, match="different size|was bfloat16"):
        plan_from_state(st, _units(as_f32), 0, None)


def test_dtype_metadata_checked_when_size_matches():
    model = W.build_mlp_stack(4, 64, 176, seed=0)
    units = _units(model)
    plan = plan_streaming(units, [u.label for u in units], None, 0, 2)
    st = state_from_plan(model, units, plan, {}, "allocation_block_transfer")
    twin = W.build_mlp_stack(4, 64, 176, seed=0)
    for p in twin.parameters():
        p.data = p.data.view(torch.float16)  # same bytes, other dtype
    with pytest.raises(ValueError, match="was bfloat16"):
        plan_from_state(st, _units(twin), 0, None)


def test_validation_catches_inconsistent_block_plan():
    model = W.build_mlp_stack(6, 64, 176, seed=0)
    units = _units(model)
    plan = plan_streaming(units, [u.label for u in units], None, 0, 2)
    good = state_from_plan(model, units, plan, {}, "allocation_block_transfer").to_dict()

    bad = json.loads(json.dumps(good))
    first = next(iter(bad["block_sizes"]))
    bad["block_sizes"][first] += 128
    with pytest.raises(ValueError, match="block_sizes"):
        TensorManagerState.from_dict(bad)

    bad = json.loads(json.dumps(good))
    label = next(iter(bad["label_to_block_id"]))
    bad["label_to_block_id"][label] = 99
    with pytest.raises(ValueError, match="label_to_block_id"):
        TensorManagerState.from_dict(bad)

    bad = json.loads(json.dumps(good))
    bad["gpu_tensors_names"] = bad["gpu_tensors_names"] + [bad["view_tensors_names"][0]]
    with pytest.raises(ValueError, match="gpu_tensors_names"):
        TensorManagerState.from_dict(bad)

    bad = json.loads(json.dumps(good))
    labels = list(bad["load_strategy"])
    bad["load_strategy"][labels[1]].append(bad["load_strategy"][labels[0]][0])
    with pytest.raises(ValueError):
        TensorManagerState.from_dict(bad)
