"""Build libpanmuon.so in-tree with hipcc for gfx950, and the host helper
extension _pm_host with g++ against torch's headers.

    python -m pan2_amd.build

The library is plain C ABI (include/panmuon.h) and links the HIP runtime by
SONAME (libamdhip64.so.7), so inside a process that already imported torch it
binds to torch's runtime; /opt/rocm/lib is the rpath fallback when loaded alone.
_pm_host (csrc/pm_host.cpp) has no device code: it fills pm_adam_tensor
descriptors from torch's tensor lists for the AdamW path.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpanmuon.so")
HOST_EXT = os.path.join(HERE, "_pm_host" + sysconfig.get_config_var("EXT_SUFFIX"))
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


def _host_cmd(src: str, out: str) -> list[str]:
    """g++ line of the _pm_host extension: torch's headers and libraries, its C++ ABI."""
    import torch
    from torch.utils.cpp_extension import include_paths

    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    return ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-DTORCH_EXTENSION_NAME=_pm_host",
            "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            f"-I{sysconfig.get_paths()['include']}", *[f"-I{p}" for p in include_paths()], src,
            f"-L{tlib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{tlib}", "-o", out]


def _start(cmd: list[str], verbose: bool) -> subprocess.Popen:
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(proc: subprocess.Popen, tmp: str, out: str, what: str) -> None:
    _, stderr = proc.communicate()
    if proc.returncode != 0:
        noise = "packed-fp32-ops"
        err = "\n".join(l for l in stderr.splitlines() if noise not in l)
        raise RuntimeError(f"{what} failed ({proc.returncode}):\n{err}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile csrc/panmuon.hip into pan2_amd/libpanmuon.so and csrc/pm_host.cpp
    into the _pm_host extension, side by side; returns the library's path."""
    lib = _start([hipcc(), *HIPCC_FLAGS, os.path.join(CSRC, "panmuon.hip"), "-o", LIB + ".tmp"], verbose)
    host = _start(_host_cmd(os.path.join(CSRC, "pm_host.cpp"), HOST_EXT + ".tmp"), verbose)
    try:
        _finish(lib, LIB + ".tmp", LIB, "hipcc")
    finally:
        _finish(host, HOST_EXT + ".tmp", HOST_EXT, "g++ (_pm_host)")
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
