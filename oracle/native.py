"""ctypes access to the C oracle ``liboracle.so`` (test infrastructure only).

``build()`` compiles ``ftx_oracle.c`` with gcc via the committed Makefile.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"


class OracleDesc(ctypes.Structure):
    _fields_ = [("src_off", ctypes.c_uint64), ("dst", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


def build() -> Path:
    subprocess.run(["make", "-B", "-C", str(ORACLE_DIR)], check=True, capture_output=True, text=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        l.oracle_packed_layout.restype = ctypes.c_uint64
        l.oracle_packed_layout.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p]
        l.oracle_pack.restype = None
        l.oracle_pack.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        l.oracle_scatter.restype = None
        l.oracle_scatter.argtypes = [ctypes.c_void_p, ctypes.POINTER(OracleDesc), ctypes.c_int]
        l.oracle_checksum64.restype = ctypes.c_uint64
        l.oracle_checksum64.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        _lib = l
    return _lib


def packed_layout(sizes, alignment: int = 128) -> tuple[list[int], int]:
    """C restatement of ``_compute_packed_byte_layout`` (utils.py:114-127)."""
    sizes = np.ascontiguousarray(np.asarray(list(sizes), dtype=np.uint64))
    offsets = np.zeros(max(1, len(sizes)), dtype=np.uint64)
    total = lib().oracle_packed_layout(sizes.ctypes.data, len(sizes), alignment, offsets.ctypes.data)
    return [int(x) for x in offsets[: len(sizes)]], int(total)


def pack(block: np.ndarray, offsets, sources) -> None:
    """C restatement of the block pack (allocation_block.py:179-181): ``block[off_i : off_i + n_i]`` =
    the storage bytes of source ``i`` (a contiguous uint8 numpy array of ``n_i`` bytes)."""
    sources = [np.ascontiguousarray(s).view(np.uint8).reshape(-1) for s in sources]
    offsets = list(offsets)
    if len(offsets) != len(sources):
        raise ValueError("one offset per source")
    for off, src in zip(offsets, sources):
        if off < 0 or off + src.nbytes > block.nbytes:
            raise ValueError(f"source of {src.nbytes} bytes at offset {off} overruns a {block.nbytes}-byte block")
    n = max(1, len(sources))
    offs = np.zeros(n, dtype=np.uint64)
    ptrs = np.zeros(n, dtype=np.uint64)
    sizes = np.zeros(n, dtype=np.uint64)
    for i, (off, src) in enumerate(zip(offsets, sources)):
        offs[i], ptrs[i], sizes[i] = off, src.ctypes.data, src.nbytes
    if not block.flags["C_CONTIGUOUS"]:
        raise ValueError("the block must be contiguous")
    lib().oracle_pack(block.ctypes.data, offs.ctypes.data, ptrs.ctypes.data, sizes.ctypes.data, len(sources))


def checksum64(data) -> int:
    """Checksum of a bytes-like / numpy uint8 array / CPU uint8 tensor."""
    if hasattr(data, "numpy"):
        data = data.contiguous().view(-1).numpy()
    arr = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else data)
    arr = arr.view(np.uint8).reshape(-1)
    return int(lib().oracle_checksum64(arr.ctypes.data, arr.nbytes))


def scatter(chunk: np.ndarray, descs, dst_arrays) -> None:
    """dst_arrays[i][0:n_i] = chunk[off_i:off_i+n_i] for descs (off_i, n_i)."""
    descs = list(descs)
    arr = (OracleDesc * max(1, len(descs)))()
    for i, ((off, n), dst) in enumerate(zip(descs, dst_arrays)):
        assert dst.nbytes >= n
        arr[i].src_off = off
        arr[i].dst = dst.ctypes.data
        arr[i].nbytes = n
    chunk = np.ascontiguousarray(chunk)
    lib().oracle_scatter(chunk.ctypes.data, arr, len(descs))
