"""Build the HIP C-ABI library ``libftx_hip.so`` in-tree for gfx950.

The library links against the HIP runtime that PyTorch ships, so that a
process which imports torch has exactly one HIP runtime and torch streams,
events and allocations are valid handles for the library.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libftx_hip.so"
SOURCES = ("ftx_runtime.hip", "ftx_kernels.hip", "ftx_gemm.hip", "ftx_staged.hip", "ftx_expcode.hip")
OFFLOAD_ARCH = "gfx950"


def _torch_lib_dir() -> str:
    import torch

    return str(Path(torch.__file__).resolve().parent / "lib")


def hipcc_command(output: Path = LIB_PATH) -> list[str]:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    torch_lib = _torch_lib_dir()
    return [
        hipcc,
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        # Keep the compiler from forming packed-fp32 instructions by itself.
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        *[str(CSRC / s) for s in SOURCES],
        "-o",
        str(output),
        f"-L{torch_lib}",
        "-lamdhip64",
        f"-Wl,-rpath,{torch_lib}",
        "-Wl,--no-undefined",
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library; always rebuilds. Returns the path of the ``.so``."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = hipcc_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    noise = "is not a recognized feature for this target"
    warnings = [ln for ln in (proc.stdout + proc.stderr).splitlines() if ln.strip() and noise not in ln]
    if warnings and verbose:
        sys.stderr.write("\n".join(warnings) + "\n")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
