"""The GEMM tile walks (pan2_amd/csrc/pm_tiles.hpp) are bijections: every
output tile of every stage is produced exactly once. The workspace layouts of
the same header are bijections whose 64-column units are contiguous blocks.
Host build of the same header with g++; CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_tile_walks_are_bijective(tmp_path):
    exe = tmp_path / "tile_order_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "pan2_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "tile_order_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "OK" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_layouts(tmp_path):
    exe = tmp_path / "layout_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "pan2_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "layout_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "OK" in out.stdout
