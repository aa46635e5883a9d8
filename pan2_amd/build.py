"""Build libpanmuon.so in-tree with hipcc for gfx950.

    python -m pan2_amd.build

The library is plain C ABI (include/panmuon.h) and links the HIP runtime by
SONAME (libamdhip64.so.7), so inside a process that already imported torch it
binds to torch's runtime; /opt/rocm/lib is the rpath fallback when loaded alone.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpanmuon.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 (v_pk_*_f32) forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wl,-rpath,/opt/rocm/lib",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; a ROCm toolchain is needed to build libpanmuon")
    return path


def _compile(src: str, out: str, verbose: bool) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, src, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "packed-fp32-ops"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile csrc/panmuon.hip into pan2_amd/libpanmuon.so; returns the
    library's path."""
    _compile(os.path.join(CSRC, "panmuon.hip"), LIB, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
