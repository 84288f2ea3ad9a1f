"""Configuration loading and the reference's convenience API (CPU).

Restates the reference's config tests (tests/unit/test_config*.py): file <
environment < keyword precedence, ``enabled`` off when only the environment
is read, INI/JSON/YAML files, text conversions, unknown ``FT_`` variables
rejected with a suggestion; plus the timing table and profiling suspension
counters.
"""

from __future__ import annotations

import json

import pytest
import torch

import flextensor_amd as ft
from flextensor_amd.config import OffloadConfig, load_config, load_config_from_env, load_config_from_file
from flextensor_amd.timing import OffloadTimingSnapshot, TrapTimingRecord, build_report


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    import os

    for k in list(os.environ):
        if k.startswith("FT_"):
            monkeypatch.delenv(k)


def test_env_only_defaults_enabled_to_false(monkeypatch):
    assert load_config_from_env().enabled is False
    monkeypatch.setenv("FT_ENABLED", "yes")
    assert load_config_from_env().enabled is True


@pytest.mark.parametrize("text,want", [("true", True), ("1", True), ("on", True), ("Y", True), ("false", False),
                                       ("0", False), ("off", False), ("No", False)])
def test_boolean_spellings(monkeypatch, text, want):
    monkeypatch.setenv("FT_PINNED_MEMORY", text)
    assert load_config_from_env().pinned_memory is want


def test_bad_boolean_names_the_variable(monkeypatch):
    monkeypatch.setenv("FT_PINNED_MEMORY", "maybe")
    with pytest.raises(ValueError, match="FT_PINNED_MEMORY=maybe"):
        load_config_from_env()


def test_none_lists_and_numbers_from_env(monkeypatch):
    monkeypatch.setenv("FT_MAX_GPU_MEM_FRACTION", "null")
    monkeypatch.setenv("FT_EXCLUDE_PATTERNS", "a.*, b.* ,")
    monkeypatch.setenv("FT_PROFILING_ITERS", "3")
    monkeypatch.setenv("FT_SHM_WAIT_TIMEOUT", "2.5")
    c = load_config_from_env()
    assert c.max_gpu_mem_fraction is None and c.exclude_patterns == ["a.*", "b.*"]
    assert c.profiling_iters == 3 and c.shm_wait_timeout == 2.5


def test_unknown_ft_variable_is_rejected_with_a_suggestion(monkeypatch):
    monkeypatch.setenv("FT_NUM_BLOKS", "3")
    with pytest.raises(ValueError, match="Did you mean: FT_NUM_BLOCKS"):
        load_config_from_env()


def test_file_then_env_then_kwargs(monkeypatch, tmp_path):
    ini = tmp_path / "ft.conf"
    ini.write_text("[flextensor]\nenabled = true\nnum_blocks = 5\ninclude_patterns = layers.*, head\n"
                   "profiling_iters = 7\n")
    c = load_config(ini)
    assert c.enabled and c.num_blocks == 5 and c.include_patterns == ["layers.*", "head"]
    monkeypatch.setenv("FT_NUM_BLOCKS", "6")
    c = load_config(ini, profiling_iters=2)
    assert c.num_blocks == 6 and c.profiling_iters == 2  # env over file, kwargs over env
    assert load_config_from_file(ini).num_blocks == 5  # no environment overrides
    monkeypatch.setenv("FT_CONFIG_FILE", str(ini))
    assert load_config().include_patterns == ["layers.*", "head"]


@pytest.mark.parametrize("suffix", [".json", ".yaml"])
def test_json_and_yaml_files(tmp_path, suffix):
    data = {"enabled": "true", "num_blocks": 3, "min_blocks": 2, "include_patterns": ["blocks.*"], "not_a_field": 1,
            "max_gpu_mem_bytes": "1024"}
    path = tmp_path / f"ft{suffix}"
    if suffix == ".json":
        path.write_text(json.dumps(data))
    else:
        import yaml

        path.write_text(yaml.safe_dump(data))
    c = load_config_from_file(path)
    assert c.enabled is True and c.num_blocks == 3 and c.min_blocks == 2 and c.include_patterns == ["blocks.*"]
    assert c.max_gpu_mem_bytes == 1024


def test_file_errors(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_config_from_file()
    with pytest.raises(FileNotFoundError):
        load_config(tmp_path / "missing.json")
    bad = tmp_path / "ft.toml"
    bad.write_text("x")
    with pytest.raises(ValueError, match="Unsupported"):
        load_config(bad)
    ini = tmp_path / "ft.ini"
    ini.write_text("[other]\nenabled=1\n")
    with pytest.raises(ValueError, match=r"\[flextensor\]"):
        load_config(ini)


def test_shm_namespace_required_when_enabled():
    with pytest.raises(ValueError, match="shm_namespace"):
        OffloadConfig(shm_enabled=True)
    assert OffloadConfig(shm_enabled=True, shm_namespace="run1").shm_namespace == "run1"


def test_timing_tables():
    snap = OffloadTimingSnapshot([TrapTimingRecord("layers.0", 2.0, 5.0, 0.0),
                                  TrapTimingRecord("layers.1", 2.0, 5.0, 0.5)])
    text = ft.format_offload_timing_table(snap)
    lines = text.splitlines()
    assert lines[0] == "Offload Timing (single pass)"
    assert any(ln.startswith("layers.1") and ln.endswith("<-") for ln in lines)  # a wait that was not hidden
    assert any(ln.startswith("Total") and "10.000" in ln and "4.000" in ln and "0.500" in ln for ln in lines)
    rep = build_report([snap, snap])
    text = ft.format_offload_timing_table(rep)
    assert text.splitlines()[0] == "Offload Timing (2 passes)"
    assert "hidden fraction 0.8750" in text  # 1 - 1.0 / 8.0
    assert ft.format_offload_timing_table(OffloadTimingSnapshot([])) == "No offload timing data."


def test_profiling_suspension_is_reference_counted():
    """tests/unit/test_profiling_control.py:67-133,409-445: control needs init() or offload() first; then
    suspensions nest, an unbalanced resume raises, and release() forgets them."""
    mgr = ft.OffloadManager("suspend-test")
    for call in (mgr.suspend_profiling, mgr.resume_profiling, mgr.clear_profiling_durations):
        with pytest.raises(RuntimeError, match=rf"{call.__name__}\(\) called before flextensor\.offload"):
            call()
    with pytest.raises(RuntimeError, match=r"pause_profiling\(\) called before flextensor\.offload"):
        with mgr.pause_profiling():
            pass
    mgr.init(OffloadConfig())
    with pytest.raises(RuntimeError, match="without a matching"):
        mgr.resume_profiling()
    mgr.suspend_profiling()
    with mgr.pause_profiling():
        assert mgr._suspend_count == 2 and mgr.is_profiling_suspended()
    assert mgr._suspend_count == 1
    mgr.resume_profiling()
    assert mgr._suspend_count == 0 and not mgr.is_profiling_suspended()
    mgr.suspend_profiling()
    mgr.release()
    assert not mgr.is_profiling_suspended()
    with pytest.raises(RuntimeError, match="called before flextensor.offload"):
        mgr.suspend_profiling()


def test_profiling_control_is_inert_when_offload_is_disabled():
    """tests/unit/test_profiling_control.py:357-400: the disabled manager accepts every call and is never
    suspended."""
    mgr = ft.OffloadManager("suspend-noop")
    model = torch.nn.Linear(2, 2)
    assert mgr.offload(model, OffloadConfig(enabled=False)) is model
    mgr.resume_profiling()  # no matching suspend needed
    mgr.suspend_profiling()
    assert not mgr.is_profiling_suspended()
    with mgr.pause_profiling() as inside:
        assert inside is None and not mgr.is_profiling_suspended()
    mgr.clear_profiling_durations()
    mgr.release()


def test_init_and_set_config_before_offload():
    ft.init(OffloadConfig(num_blocks=6), name="init-test")
    assert ft.get_offload_manager("init-test").config.num_blocks == 6
    ft.set_config(OffloadConfig(num_blocks=5), name="init-test")
    assert ft.get_offload_manager("init-test").config.num_blocks == 5
    assert ft.offload_units("init-test") == () and ft.resident_units("init-test") == ()
    ft.release("init-test")
