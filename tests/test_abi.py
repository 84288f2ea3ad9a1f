"""The C-ABI library loads without a GPU and exports every declared entry point."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

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


def test_arena_register_is_refused_in_c_without_the_runtime():
    """In-place page-locking is refused by the C entry point itself, for any input, before any runtime call
    (host_pinning.py:206-265 is the reference's pin_in_place it stands in for): a C caller that binds
    ``pin_in_place`` to it gets FTX_ERR_UNSUPPORTED on a box with no GPU at all."""
    import ctypes

    from flextensor_amd import _native

    lib = _native.load()
    buf = ctypes.create_string_buffer(1 << 16)
    for ptr, n in ((ctypes.addressof(buf), 1 << 16), (None, 0), (ctypes.addressof(buf), 1)):
        assert lib.ftx_arena_register(ptr, n, 0) == _native.FTX_ERR_UNSUPPORTED
        assert b"refused in this build" in lib.ftx_last_error()
    assert lib.ftx_arena_unregister(ctypes.addressof(buf)) == _native.FTX_ERR_INVALID
    with pytest.raises(_native.FtxError, match="refused in this build") as info:
        _native.arena_register(ctypes.addressof(buf), 1 << 16)
    assert info.value.code == _native.FTX_ERR_UNSUPPORTED


def test_a_per_call_copy_policy_is_checked_before_any_device_call():
    """``ftx_copy_h2d_policy`` validates the caller's policy first: out-of-range values are refused with no
    device present, and the library default is not changed by a per-call policy."""
    import ctypes

    from flextensor_amd import _native

    lib = _native.load()
    before = _native.get_copy_policy()
    for bad in (_native.copy_policy(0, 0, 0, 0), _native.copy_policy(0, 0, 9, 0), _native.copy_policy(0, 0, 1, -1),
                _native.copy_policy(0, 0, 1, (1 << 20) + 1)):
        assert lib.ftx_copy_h2d_policy(None, None, 0, _native.COPY_SDMA, ctypes.byref(bad), None) == \
            _native.FTX_ERR_INVALID
    with pytest.raises(_native.FtxError, match="n_copy_streams"):
        _native.copy_h2d(0, 0, 0, _native.COPY_AUTO, 0, _native.copy_policy(0, 0, 0, 0))
    # a valid policy and nothing to copy: done without touching a device
    _native.copy_h2d(0, 0, 0, _native.COPY_AUTO, 0, _native.copy_policy(1 << 30, 1, 8, 8))
    assert _native.get_copy_policy() == before
    p = _native.copy_policy(5, 2**64, 2, 3)  # above the 64-bit range reads as "never split"
    assert p.astuple() == (5, 2**64 - 1, 2, 3) and p == _native.copy_policy(5, 2**64 - 1, 2, 3)


def _run_python(code: str) -> "subprocess.CompletedProcess":
    import subprocess
    import sys

    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                          cwd=str(ROOT))


def test_shutdown_is_idempotent_and_refuses_later_work():
    """``ftx_shutdown`` (core/transfer.py:133-142: synchronize, then refuse further work) releases the
    library's own resources once; a second call is a no-op; afterwards calls that would start work or
    allocate fail with FTX_ERR_UNSUPPORTED and a message, and calls that release handles still succeed.
    Run in a child process: a shut-down library stays shut down for the rest of its process."""
    code = (
        "import ctypes\n"
        "import flextensor_amd._native as nat\n"
        "lib = nat.load()\n"
        "src, dst = ctypes.create_string_buffer(8 << 20), ctypes.create_string_buffer(8 << 20)\n"
        "nat.host_memcpy(ctypes.addressof(dst), ctypes.addressof(src), 8 << 20)  # starts the host thread pool\n"
        "assert lib.ftx_shutdown() == 0 and lib.ftx_shutdown() == 0\n"
        "nat.shutdown()\n"
        "refused = {\n"
        "  'host_memcpy': lib.ftx_host_memcpy(ctypes.addressof(dst), ctypes.addressof(src), 64),\n"
        "  'copy_h2d': lib.ftx_copy_h2d(None, None, 0, 0, None),\n"
        "  'arena_alloc': lib.ftx_arena_alloc(4096, 0, ctypes.byref(ctypes.c_void_p())),\n"
        "  'event_create': lib.ftx_event_create(0, ctypes.byref(ctypes.c_void_p())),\n"
        "  'scatter': lib.ftx_scatter(None, None, 0, None),\n"
        "  'fp8_linear': lib.ftx_fp8_linear(None, None, None, None, 0, 0, 0, None, 0, None),\n"
        "}\n"
        "assert all(rc == nat.FTX_ERR_UNSUPPORTED for rc in refused.values()), refused\n"
        "assert b'shut down' in lib.ftx_last_error()\n"
        "released = [lib.ftx_event_destroy(None), lib.ftx_stream_destroy(None), lib.ftx_arena_free(None),\n"
        "            lib.ftx_device_free(None), lib.ftx_scatter_plan_destroy(None)]\n"
        "assert released == [0] * 5, released\n"
        "print('shut down')\n"
    )
    out = _run_python(code)
    assert out.returncode == 0 and out.stdout.strip() == "shut down", out.stdout + out.stderr


def test_exit_releases_the_library_quietly():
    """At interpreter exit the binding calls ``ftx_shutdown`` ahead of torch's exit handlers: a process whose
    host thread pool is running exits with status 0 and nothing on stderr. Exit handlers run last-registered
    first, so a probe registered before the binding is imported runs after its shutdown (and is refused),
    and one registered after it runs before (and still works)."""
    code = (
        "import atexit, ctypes\n"
        "held = {}\n"
        "def probe(when):\n"
        "    rc = held['lib'].ftx_host_memcpy(ctypes.addressof(held['dst']), ctypes.addressof(held['src']), 64)\n"
        "    print(when, 'refused' if rc == 4 else 'live', flush=True)\n"
        "atexit.register(probe, 'after')\n"
        "import flextensor_amd._native as nat\n"
        "held['lib'] = nat.load()\n"
        "held['src'], held['dst'] = ctypes.create_string_buffer(32 << 20), ctypes.create_string_buffer(32 << 20)\n"
        "nat.host_memcpy(ctypes.addressof(held['dst']), ctypes.addressof(held['src']), 32 << 20)\n"
        "atexit.register(probe, 'before')\n"
    )
    out = _run_python(code)
    assert out.returncode == 0 and out.stderr == "", out.stderr
    assert out.stdout.split() == ["before", "live", "after", "refused"], out.stdout


def test_event_flags_are_checked_before_the_runtime():
    """``ftx_event_create`` takes FTX_EVENT_TIMING and FTX_EVENT_DEVICE_ONLY; any other bit is refused on the
    host, with no device involved."""
    import ctypes

    from flextensor_amd import _native

    lib = _native.load()
    ev = ctypes.c_void_p()
    for bad in (4, 8, 0x20000000, 0x80000003):
        assert lib.ftx_event_create(bad, ctypes.byref(ev)) == _native.FTX_ERR_INVALID
        assert b"unknown event flags" in lib.ftx_last_error()
    assert (_native.EVENT_TIMING, _native.EVENT_DEVICE_ONLY) == (1, 2)
