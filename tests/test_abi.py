"""The C-ABI library loads without a GPU and exports every declared entry point."""

from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions() -> list[str]:
    text = (ROOT / "include" / "ftx.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ftx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_core_entry_points():
    names = _declared_functions()
    for required in ("ftx_arena_alloc", "ftx_copy_h2d", "ftx_scatter", "ftx_event_record", "ftx_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from flextensor_amd import _native

    lib = _native.load()
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert missing == []
    assert _native.version() == 1


def test_binding_covers_every_declared_symbol():
    from flextensor_amd import _native

    assert sorted(_native.exported_symbols()) == _declared_functions()


def test_error_path_without_device_call():
    from flextensor_amd import _native

    lib = _native.load()
    rc = lib.ftx_set_copy_policy(0, 0, 99, 0)
    assert rc == _native.FTX_ERR_INVALID
    assert b"n_copy_streams" in lib.ftx_last_error()
