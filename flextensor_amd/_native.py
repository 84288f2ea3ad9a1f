"""ctypes binding of ``libftx_hip.so`` (the C ABI declared in ``include/ftx.h``).

``import torch`` happens before the library is loaded so that the library
binds to the HIP runtime torch already loaded (one runtime per process).
Every wrapper raises :class:`FtxError` with the library's message when a call
fails. There is no fallback: if the library is missing the first use raises
:class:`FtxLibraryMissing`.
"""

from __future__ import annotations

import atexit
import ctypes
import os
import sys
import threading
from pathlib import Path

import torch  # noqa: F401  - must be loaded before the library (shared HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "libftx_hip.so"

FTX_OK = 0
FTX_ERR_INVALID = 1
FTX_ERR_HIP = 2
FTX_ERR_OOM = 3
FTX_ERR_UNSUPPORTED = 4

COPY_SDMA = 0
COPY_KERNEL = 1
COPY_AUTO = 2
COPY_STAGED = 3
COPY_MODES = {"sdma": COPY_SDMA, "kernel": COPY_KERNEL, "auto": COPY_AUTO, "staged": COPY_STAGED}

ARENA_DEFAULT = 0
ARENA_COHERENT = 1
ARENA_NONCOHERENT = 2
ARENA_WRITECOMBINED = 4
ARENA_NUMA_USER = 8

EVENT_DEFAULT = 0
EVENT_TIMING = 1
EVENT_DEVICE_ONLY = 2


class FtxError(RuntimeError):
    """A C-ABI call failed; ``code`` is the FTX_ERR_* status."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(message)
        self.code = code


class FtxOutOfMemoryError(FtxError, MemoryError):
    """Host or device allocation failed inside the library."""


class FtxLibraryMissing(ImportError):
    """``libftx_hip.so`` has not been built."""


class FtxDesc(ctypes.Structure):
    """Mirror of ``ftx_desc``: dst[0:nbytes) = chunk[src_off:src_off+nbytes)."""

    _fields_ = [("src_off", ctypes.c_uint64), ("dst", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class CopyPolicy(ctypes.Structure):
    """Mirror of ``ftx_copy_policy``: a copy policy a caller owns and passes with each copy.

    ``kernel_max_bytes``: chunks up to this go to the zero-copy kernel under
    ``COPY_AUTO``; ``split_min_bytes``: SDMA copies from this size up are split
    over ``n_copy_streams`` (1..8); ``kernel_grid``: zero-copy workgroups (0 is
    the library's default, 64).
    """

    _fields_ = [("kernel_max_bytes", ctypes.c_uint64), ("split_min_bytes", ctypes.c_uint64),
                ("n_copy_streams", ctypes.c_int32), ("kernel_grid", ctypes.c_int32)]

    def astuple(self) -> tuple[int, int, int, int]:
        return (int(self.kernel_max_bytes), int(self.split_min_bytes), int(self.n_copy_streams),
                int(self.kernel_grid))

    def __eq__(self, other: object) -> bool:
        return isinstance(other, CopyPolicy) and self.astuple() == other.astuple()

    def __repr__(self) -> str:
        km, sm, ns, kg = self.astuple()
        return f"CopyPolicy(kernel_max_bytes={km}, split_min_bytes={sm}, n_copy_streams={ns}, kernel_grid={kg})"


def copy_policy(kernel_max_bytes: int, split_min_bytes: int, n_copy_streams: int, kernel_grid: int = 0) -> CopyPolicy:
    """A :class:`CopyPolicy`; ``split_min_bytes`` above the 64-bit range means "never split"."""
    return CopyPolicy(int(kernel_max_bytes), min(int(split_min_bytes), 2**64 - 1), int(n_copy_streams),
                      int(kernel_grid))


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int
_uint = ctypes.c_uint

# name -> (argtypes); every function returns int except ftx_last_error / ftx_version.
_SIGNATURES: dict[str, list] = {
    "ftx_device_count": [ctypes.POINTER(_int)],
    "ftx_set_device": [_int],
    "ftx_get_device": [ctypes.POINTER(_int)],
    "ftx_device_synchronize": [],
    "ftx_device_info": [ctypes.POINTER(_int), ctypes.POINTER(_int), ctypes.POINTER(_sz)],
    "ftx_arena_alloc": [_sz, _uint, ctypes.POINTER(_vp)],
    "ftx_arena_free": [_vp],
    "ftx_arena_register": [_vp, _sz, _uint],
    "ftx_arena_unregister": [_vp],
    "ftx_host_device_ptr": [_vp, ctypes.POINTER(_vp)],
    "ftx_device_alloc": [_sz, ctypes.POINTER(_vp)],
    "ftx_device_free": [_vp],
    "ftx_memset_async": [_vp, _int, _sz, _vp],
    "ftx_copy_d2h": [_vp, _vp, _sz, _vp],
    "ftx_stream_create": [ctypes.POINTER(_vp)],
    "ftx_stream_destroy": [_vp],
    "ftx_stream_synchronize": [_vp],
    "ftx_stream_query": [_vp, ctypes.POINTER(_int)],
    "ftx_event_create": [_uint, ctypes.POINTER(_vp)],
    "ftx_event_destroy": [_vp],
    "ftx_event_record": [_vp, _vp],
    "ftx_timestamp": [_vp, _vp],
    "ftx_wall_clock_khz": [ctypes.POINTER(ctypes.c_int)],
    "ftx_stream_wait_event": [_vp, _vp],
    "ftx_event_query": [_vp, ctypes.POINTER(_int)],
    "ftx_event_synchronize": [_vp],
    "ftx_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(ctypes.c_float)],
    "ftx_copy_h2d": [_vp, _vp, _sz, _int, _vp],
    "ftx_copy_h2d_policy": [_vp, _vp, _sz, _int, ctypes.POINTER(CopyPolicy), _vp],
    "ftx_shutdown": [],
    "ftx_set_copy_policy": [_sz, _sz, _int, _int],
    "ftx_get_copy_policy": [ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(_int), ctypes.POINTER(_int)],
    "ftx_scatter_plan_create": [ctypes.POINTER(FtxDesc), _int, _sz, ctypes.POINTER(_vp)],
    "ftx_scatter_plan_destroy": [_vp],
    "ftx_scatter_plan_info": [_vp, ctypes.POINTER(_int), ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint64)],
    "ftx_scatter_run": [_vp, _vp, _vp],
    "ftx_scatter": [_vp, ctypes.POINTER(FtxDesc), _int, _vp],
    "ftx_checksum64": [_vp, _sz, _vp, ctypes.POINTER(ctypes.c_uint64)],
    "ftx_set_staging_policy": [_sz, _int],
    "ftx_get_staging_policy": [ctypes.POINTER(_sz), ctypes.POINTER(_int)],
    "ftx_host_memcpy": [_vp, _vp, _sz],
    "ftx_fp8_linear_workspace": [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(_sz)],
    "ftx_fp8_linear": [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp, _sz, _vp],
    "ftx_fp8_linear_static": [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp],
    "ftx_hbm_read_probe": [_vp, _sz, _vp, ctypes.c_int, _vp],
    "ftx_mfma_probe": [ctypes.c_int, ctypes.c_int, _vp, _vp],
    "ftx_mfma_probe_shape": [ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp],
    "ftx_fp8_linear_group_workspace": [ctypes.c_int64, _vp, ctypes.c_int, ctypes.c_int64, ctypes.POINTER(_sz)],
    "ftx_fp8_linear_group": [_vp, ctypes.c_int, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _sz, _vp],
    "ftx_set_fp8_linear_config": [_int, _int],
    "ftx_fp8_linear_fused_workspace": [ctypes.c_int64, _vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                       ctypes.POINTER(_sz)],
    "ftx_expcode_encode": [_vp, _sz, _vp, _sz, ctypes.POINTER(_sz)],
    "ftx_expcode_raw_bytes": [_vp, _sz, ctypes.POINTER(_sz)],
    "ftx_expcode_decode_h2d": [_vp, _vp, _sz, ctypes.POINTER(CopyPolicy), _vp],
    "ftx_expcode_decode_d2d": [_vp, _vp, _sz, _sz, ctypes.c_int, _vp],
    "ftx_expcode_encode_dense": [_vp, _sz, _vp, _sz, ctypes.POINTER(_sz)],
    "ftx_expcode_decode_dense_d2d": [_vp, _vp, _sz, _sz, ctypes.c_int, _vp],
    "ftx_fp8_linear_fused": [_vp, ctypes.c_int, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _vp,
                             _vp, _sz, _vp],
}

FP8_EPILOGUE_NONE = 0
FP8_EPILOGUE_SWIGLU = 1
FP8_EPILOGUE_RESIDUAL = 2

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()
# Finalizers stop releasing handles once the interpreter is shutting down:
# the HIP runtime may already be torn down by then.
_alive = True


def _mark_exit() -> None:
    """At interpreter exit: stop finalizers from releasing handles, then let the library release what it
    holds (``ftx_shutdown``: wait for the devices, join its host threads, free its staging buffers, copy
    streams and events) while the HIP runtime is still up. Registered after ``import torch``, so it runs
    ahead of torch's own exit handlers."""
    global _alive
    _alive = False
    if _lib is not None:
        rc = _lib.ftx_shutdown()
        if rc != FTX_OK:  # the process is ending either way; say what could not be released
            msg = (_lib.ftx_last_error() or b"").decode(errors="replace")
            print(f"flextensor_amd: ftx_shutdown at exit returned {rc}: {msg}", file=sys.stderr, flush=True)


atexit.register(_mark_exit)


def shutdown() -> None:
    """``ftx_shutdown``: release the library's own resources now; later work is refused (idempotent)."""
    call("ftx_shutdown")


def live() -> bool:
    """Whether handles may still be released (library loaded, not exiting)."""
    return _lib is not None and _alive


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load the library once and declare its signatures."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        lib_path = Path(path) if path is not None else LIB_PATH
        if not lib_path.exists():
            raise FtxLibraryMissing(
                f"{lib_path} is missing; build it with `python -m flextensor_amd._build` "
                "(hipcc, --offload-arch=gfx950)"
            )
        lib = ctypes.CDLL(str(lib_path))
        lib.ftx_last_error.restype = ctypes.c_char_p
        lib.ftx_last_error.argtypes = []
        lib.ftx_version.restype = ctypes.c_int
        lib.ftx_version.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


def check(rc: int) -> None:
    """Raise the FtxError matching a non-zero status."""
    if rc == FTX_OK:
        return
    msg = (lib().ftx_last_error() or b"").decode(errors="replace")
    if rc == FTX_ERR_OOM:
        raise FtxOutOfMemoryError(rc, msg)
    raise FtxError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


# ---- convenience wrappers ---------------------------------------------------


def version() -> int:
    return int(lib().ftx_version())


def device_count() -> int:
    n = ctypes.c_int(0)
    call("ftx_device_count", ctypes.byref(n))
    return n.value


def device_info() -> tuple[int, int, int]:
    cu, xcd, mem = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_size_t(0)
    call("ftx_device_info", ctypes.byref(cu), ctypes.byref(xcd), ctypes.byref(mem))
    return cu.value, xcd.value, mem.value


def arena_alloc(nbytes: int, flags: int = ARENA_DEFAULT) -> int:
    p = ctypes.c_void_p()
    call("ftx_arena_alloc", nbytes, flags, ctypes.byref(p))
    return int(p.value)


def arena_free(ptr: int) -> None:
    call("ftx_arena_free", ptr)


HOST_REGISTER_REFUSED = (
    "in-place page-locking (pinned_memory_mode='host_register', hipHostRegister of existing memory) is refused "
    "in this build: the MI355X hosts it targets reject hipHostRegister, and the failed call's error can surface "
    "in the next GPU call. Use pinned_memory_mode='torch' (blocks are allocated directly in page-locked arenas); "
    "shared-memory blocks then stream through the staged copy engine.")


def arena_register(ptr: int, nbytes: int, flags: int = 0) -> None:
    """Page-lock existing host memory in place: refused in this build.

    ``ftx_arena_register`` returns ``FTX_ERR_UNSUPPORTED`` for every input
    without calling the runtime; this raises that as :class:`FtxError`.
    """
    call("ftx_arena_register", ptr, nbytes, flags)
    raise AssertionError("ftx_arena_register accepted a registration it is built to refuse")


def arena_unregister(ptr: int) -> None:
    call("ftx_arena_unregister", ptr)


def host_device_ptr(ptr: int) -> int:
    d = ctypes.c_void_p()
    call("ftx_host_device_ptr", ptr, ctypes.byref(d))
    return int(d.value)


def stream_create() -> int:
    s = ctypes.c_void_p()
    call("ftx_stream_create", ctypes.byref(s))
    return int(s.value)


def event_create(flags: int = EVENT_DEFAULT) -> int:
    e = ctypes.c_void_p()
    call("ftx_event_create", flags, ctypes.byref(e))
    return int(e.value)


def event_elapsed_ms(start: int, end: int) -> float:
    ms = ctypes.c_float(0.0)
    call("ftx_event_elapsed_ms", start, end, ctypes.byref(ms))
    return float(ms.value)


def event_query(event: int) -> bool:
    done = ctypes.c_int(0)
    call("ftx_event_query", event, ctypes.byref(done))
    return bool(done.value)


def copy_h2d(dst: int, src: int, nbytes: int, mode: int, stream: int, policy: CopyPolicy | None = None) -> None:
    """Host-to-device copy; ``policy`` None copies under the library default (``set_copy_policy``)."""
    if policy is None:
        call("ftx_copy_h2d", dst, src, nbytes, mode, stream)
    else:
        call("ftx_copy_h2d_policy", dst, src, nbytes, mode, ctypes.byref(policy), stream)


def set_copy_policy(kernel_max_bytes: int, split_min_bytes: int, n_copy_streams: int, kernel_grid: int = 0) -> None:
    call("ftx_set_copy_policy", kernel_max_bytes, split_min_bytes, n_copy_streams, kernel_grid)


def get_copy_policy() -> tuple[int, int, int, int]:
    a, b, c, d = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_int(0), ctypes.c_int(0)
    call("ftx_get_copy_policy", ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), ctypes.byref(d))
    return a.value, b.value, c.value, d.value


def make_desc_array(descs) -> ctypes.Array:
    """Build a ctypes ``ftx_desc[]`` from (src_off, dst, nbytes) triples."""
    descs = list(descs)
    arr = (FtxDesc * max(1, len(descs)))()
    for i, (off, dst, n) in enumerate(descs):
        arr[i].src_off = off
        arr[i].dst = dst
        arr[i].nbytes = n
    return arr


def checksum64(dev_ptr: int, nbytes: int, stream: int) -> int:
    out = ctypes.c_uint64(0)
    call("ftx_checksum64", dev_ptr, nbytes, stream, ctypes.byref(out))
    return int(out.value)


def exported_symbols() -> list[str]:
    """Names of the C entry points this binding declares."""
    return ["ftx_last_error", "ftx_version", *_SIGNATURES.keys()]


def set_staging_policy(piece_bytes: int, n_threads: int = 0) -> None:
    call("ftx_set_staging_policy", piece_bytes, n_threads)


def get_staging_policy() -> tuple[int, int]:
    piece, threads = _sz(0), _int(0)
    call("ftx_get_staging_policy", ctypes.byref(piece), ctypes.byref(threads))
    return int(piece.value), int(threads.value)


def host_memcpy(dst: int, src: int, nbytes: int) -> None:
    """Parallel host copy of ``nbytes`` (the staged engine's thread pool)."""
    call("ftx_host_memcpy", dst, src, nbytes)
