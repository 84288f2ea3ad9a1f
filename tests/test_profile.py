"""Saved profiles (schema 3): JSON shape, consistency checks, plan round trip.

The fixtures marked with a reference location are transcribed from the
reference's own tests; the round trip checks that a plan written by
:func:`state_from_plan` and read back by :func:`plan_from_state` gives the
same slot plan, streamed set and loader order as the planner produced.
"""

from __future__ import annotations

import json

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
