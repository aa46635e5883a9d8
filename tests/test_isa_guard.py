"""Static checks of the GEMM kernels' gfx950 assembly (CPU only; hipcc -S).

The GEMM engine issues its MFMAs from inline asm with the accumulators tied
in AGPRs, so the compiler does not know their latency. Three things would
then corrupt results silently, and none may appear in any GEMM instantiation:
  * scratch traffic (a spill of an accumulator right after its MFMA reads a
    stale value, and spills of anything cost bandwidth),
  * accumulator copies (v_accvgpr_read/write/mov) between the first and the
    last MFMA,
  * a load whose destination is a source register of one of the previous 8
    MFMAs inside the MFMA region (an MFMA reads its sources when it executes,
    after issue).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "pan2_amd", "csrc", "panmuon.hip")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("needs hipcc")
    out = tmp_path_factory.mktemp("isa") / "panmuon.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "--cuda-device-only", "-S", SRC, "-o", str(out)],
                   check=True, capture_output=True)
    return out.read_text()


@pytest.fixture(scope="module")
def gemm_kernels(asm):
    kernels = {}
    for m in re.finditer(r"^(_ZN2pm17pm_ns_gemm_kernel\w+):.*$", asm, flags=re.M):
        body = asm[m.end():]
        kernels[m.group(1)] = body[:body.index("s_endpgm")].split("\n")
    # panel layout: GRAM, POLY, UPDATE, FINAL x {f32, bf16}, each also as its
    # K-split instantiation (chunk partials instead of the epilogue); row-major:
    # GRAM, POLY (pm_gram, pm_gemm_symmetric)
    assert len(kernels) == 12, sorted(kernels)
    assert sum(1 for k in kernels if k.endswith("ELb1EEEvNS_8GemmArgsE")) == 5, sorted(kernels)
    return kernels


@pytest.fixture(scope="module")
def reduce_kernels(asm):
    kernels = {}
    for m in re.finditer(r"^(_ZN2pm19pm_ns_reduce_kernel\w+):.*$", asm, flags=re.M):
        body = asm[m.end():]
        kernels[m.group(1)] = body[:body.index("s_endpgm")].split("\n")
    assert len(kernels) == 5, sorted(kernels)  # GRAM, POLY, UPDATE, FINAL x {f32, bf16}
    return kernels


def test_reduce_kernels_have_no_scratch(reduce_kernels):
    for name, lines in reduce_kernels.items():
        n = sum(1 for ln in lines if "scratch_" in ln)
        assert n == 0, f"{name}: {n} scratch instructions"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def test_no_scratch(gemm_kernels):
    for name, lines in gemm_kernels.items():
        n = sum(1 for ln in lines if "scratch_" in ln)
        assert n == 0, f"{name}: {n} scratch instructions"


def test_no_accumulator_copies_between_mfmas(gemm_kernels):
    for name, lines in gemm_kernels.items():
        idx = [i for i, ln in enumerate(lines) if "v_mfma" in ln]
        copies = [ln.strip() for ln in lines[idx[0]:idx[-1]] if "v_accvgpr" in ln]
        assert not copies, f"{name}: {len(copies)} accumulator copies in the MFMA region, e.g. {copies[:2]}"


def test_loads_do_not_overwrite_queued_mfma_sources(gemm_kernels):
    for name, lines in gemm_kernels.items():
        idx = [i for i, ln in enumerate(lines) if "v_mfma" in ln]
        recent = []
        for ln in lines[idx[0]:idx[-1] + 1]:
            t = ln.strip()
            if t.startswith("v_mfma"):
                ops = [o.strip() for o in t.split(None, 1)[1].split(",")]
                recent = (recent + [_regs(ops[1]) | _regs(ops[2])])[-8:]
            elif t.startswith("ds_read") or t.startswith("global_load") or (
                    t.startswith("buffer_load") and " lds" not in t):
                dst = _regs(t.split(None, 1)[1].split(",")[0].strip())
                assert not any(dst & src for src in recent), f"{name}: {t}"


def test_no_scalar_memory_writes(gemm_kernels):
    """Every store and atomic goes through the vector memory path (the tile
    queues' counters included)."""
    bad = re.compile(r"^\s*(s_store|s_buffer_store|s_atomic|s_buffer_atomic|s_scratch_store|s_dcache_wb)")
    for name, lines in gemm_kernels.items():
        hits = [ln.strip() for ln in lines if bad.match(ln)]
        assert not hits, f"{name}: {hits[:2]}"


def test_small_kernels_keep_lds_in_lds(asm):
    """The small-matrix kernels hold their LDS addresses in registers: no
    scratch traffic, and the core kernel's M x M products read and write LDS
    with ds_ instructions (a pointer that went through memory turns them into
    flat accesses that wait on both counters). The apply that also forms the
    gram writes and reads its X' tiles with ds_ instructions: a flat access
    there would also count in vmcnt, whose exact waits the apply relies on.
    The prologue that forms the first gram writes its X units to LDS and reads
    the MFMA fragments back with ds_ instructions."""
    kernels = {}
    for m in re.finditer(r"^(_ZN2pm\d+pm_small_\w+):.*$", asm, flags=re.M):
        body = asm[m.end():]
        kernels[m.group(1)] = body[:body.index(".Lfunc_end")]
    assert len(kernels) == 10, sorted(kernels)
    for name, body in kernels.items():
        assert "scratch_" not in body, name
        if "core_kernel" in name:
            wide_flat = re.findall(r"^\s*flat_(load|store)_dwordx[24]", body, flags=re.M)
            assert not wide_flat, f"{name}: {len(wide_flat)} flat accesses of 8 or 16 bytes"
            assert "ds_read_b128" in body, name
        if "prologue_kernel" in name:
            assert "ds_write_b128" in body and "ds_read_b128" in body and "v_mfma" in body, name
    gram_apply = [name for name in kernels if "apply_kernelILi2ELi1ELb1E" in name]
    assert len(gram_apply) == 1, sorted(kernels)
    body = kernels[gram_apply[0]]
    assert not re.findall(r"^\s*flat_", body, flags=re.M), gram_apply[0]
    assert "ds_write_b64" in body and "ds_read_b128" in body, gram_apply[0]
