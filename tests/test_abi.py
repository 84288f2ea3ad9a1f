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


def test_missing_library_fails_loudly():
    """With no built library the product refuses to run: the first native call raises
    FtxLibraryMissing (an ImportError); nothing falls back to a host path or to the oracle."""
    import subprocess
    import sys

    code = (
        "from pathlib import Path\n"
        "import flextensor_amd._native as nat\n"
        "nat.LIB_PATH = Path('/nonexistent/libftx_hip.so')\n"
        "for attempt in (lambda: nat.load(), lambda: nat.checksum64(0, 0, 0),\n"
        "                lambda: nat.call('ftx_scatter', None, None, 0, None)):\n"
        "    try:\n"
        "        attempt()\n"
        "    except nat.FtxLibraryMissing as e:\n"
        "        assert isinstance(e, ImportError) and 'libftx_hip.so is missing' in str(e)\n"
        "    else:\n"
        "        raise SystemExit('a native call ran without the library')\n"
        "import sys\n"
        "assert not any(m == 'oracle' or m.startswith('oracle.') for m in sys.modules), 'oracle imported'\n"
        "print('refused')\n"
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                         cwd=str(Path(__file__).resolve().parents[1]))
    assert out.returncode == 0 and out.stdout.strip().endswith("refused"), out.stdout + out.stderr
