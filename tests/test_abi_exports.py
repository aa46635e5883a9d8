"""libpanmuon's C ABI on the CPU: the library loads, exports exactly what
include/panmuon.h declares, its structs have the header's layout, and argument
errors come back as the documented return codes. No call here reaches the
device: every case fails (or returns) in host-side validation.
"""
import ctypes
import os
import re
import shutil
import subprocess
import sys

import pytest

from pan2_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "panmuon.h")


def _ensure_built():
    if not os.path.exists(_lib.LIB_PATH):
        from pan2_amd.build import build

        build()
    return _lib.load()


@pytest.fixture(scope="module")
def lib():
    return _ensure_built()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"(?:int|size_t|const\s+char\s*\*)\s+(pm_\w+)\s*\(", text))


def test_header_declares_what_the_binding_binds():
    assert header_functions() == set(_lib.EXPORTS)


def test_library_exports_every_header_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                             check=True).stdout
        exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
        pm_syms = {s for s in exported if s.startswith("pm_")}
        assert pm_syms == header_functions(), pm_syms ^ header_functions()


def test_abi_version(lib):
    text = open(HEADER).read()
    want = int(re.search(r"#define PM_ABI_VERSION (\d+)", text).group(1))
    assert lib.pm_abi_version() == want == _lib.ABI_VERSION


STRUCTS = {
    "pm_matrix": _lib.PmMatrix,
    "pm_ns_matrix": _lib.PmNsMatrix,
    "pm_hparams": _lib.PmHparams,
    "pm_launch_time": _lib.PmLaunchTime,
    "pm_adam_tensor": _lib.PmAdamTensor,
    "pm_adam_hparams": _lib.PmAdamHparams,
}
# ctypes field name -> C field name where Python needs another spelling
RENAME = {"in_": "in"}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc to read the C layout")
def test_struct_layout_matches_header(tmp_path):
    """Compile a C program against the header and compare every offset and size
    with the ctypes mirror."""
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "panmuon.h"', "int main(void) {"]
    for cname, cls in STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            cf = RENAME.get(f, f)
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {cf}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    seen = 0
    for line in filter(None, out):
        cname, field, value = line.split()
        cls = STRUCTS[cname]
        want = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert int(value) == want, (cname, field, value, want)
        seen += 1
    assert seen == sum(len(c._fields_) + 1 for c in STRUCTS.values())


# ---------------------------------------------------------------- host-side validation

FAKE = 0x100000  # never dereferenced: every call below fails or returns before device work


def mat(rows=256, cols=512, pdt=1, gdt=1, mdt=0, ld=None, ptrs=(FAKE, FAKE, FAKE)):
    m = _lib.PmMatrix()
    m.param, m.grad, m.momentum = ptrs
    m.rows, m.cols = rows, cols
    m.param_ld = m.grad_ld = m.momentum_ld = cols if ld is None else ld
    m.param_dtype, m.grad_dtype, m.momentum_dtype = pdt, gdt, mdt
    m.adj_ratio = 1.0
    return m


def hparams(**kw):
    hp, keep = _lib.make_hparams(**kw)
    return hp


def arr(*ms):
    return (_lib.PmMatrix * len(ms))(*ms)


def step(lib, ms, hp=None, ws=FAKE, ws_bytes=1 << 40):
    hp = hp or hparams()
    a = arr(*ms) if ms else None
    return lib.pm_muon_step(a, len(ms), ctypes.byref(hp), None, 0.02, ws, ws_bytes, None)


def test_muon_step_argument_errors(lib):
    assert step(lib, []) == 0  # nothing to do
    assert step(lib, [mat()], hparams(ns_steps=0)) == _lib.PM_EUNSUPPORTED
    assert step(lib, [mat()], hparams(ns_steps=100)) == _lib.PM_EUNSUPPORTED
    assert "ns_steps" in _lib.last_error()
    assert step(lib, [mat()], hparams(eps=-1.0)) == _lib.PM_EINVAL
    assert step(lib, [mat(rows=0)]) == _lib.PM_EINVAL
    assert step(lib, [mat(pdt=7)]) == _lib.PM_EDTYPE
    assert step(lib, [mat(ld=100)]) == _lib.PM_EINVAL
    assert "row stride" in _lib.last_error()
    assert step(lib, [mat(ptrs=(FAKE, 0, FAKE))]) == _lib.PM_EINVAL
    assert step(lib, [mat()], ws=0) == _lib.PM_EINVAL
    assert step(lib, [mat()], ws=FAKE + 8) == _lib.PM_EINVAL
    assert "aligned" in _lib.last_error()
    assert step(lib, [mat()], ws_bytes=4096) == _lib.PM_EWORKSPACE
    assert lib.pm_muon_step(None, 3, ctypes.byref(hparams()), None, 0.02, FAKE, 1 << 40, None) == _lib.PM_EINVAL
    assert lib.pm_muon_step(arr(mat()), 1, None, None, 0.02, FAKE, 1 << 40, None) == _lib.PM_EINVAL


def test_elementwise_and_gram_argument_errors(lib):
    assert lib.pm_momentum_nesterov(FAKE, 0, FAKE, 0, FAKE, 0, -1, 0.95, 1, None) == _lib.PM_EINVAL
    assert lib.pm_momentum_nesterov(FAKE, 0, FAKE, 0, FAKE, 0, 0, 0.95, 1, None) == 0
    assert lib.pm_momentum_nesterov(FAKE, 3, FAKE, 0, FAKE, 0, 16, 0.95, 1, None) == _lib.PM_EDTYPE
    assert lib.pm_momentum_nesterov(None, 0, FAKE, 0, FAKE, 0, 16, 0.95, 1, None) == _lib.PM_EINVAL
    assert lib.pm_step_param(FAKE, 0, FAKE, 0, -5, None, 0.02, 0.01, 1.0, None) == _lib.PM_EINVAL
    assert lib.pm_step_param(FAKE, 0, FAKE, 9, 16, None, 0.02, 0.01, 1.0, None) == _lib.PM_EDTYPE
    ws = lib.pm_gram_workspace_bytes()
    assert ws > 0
    assert lib.pm_gram(FAKE, 256, 320, FAKE, FAKE, ws, None) == _lib.PM_EINVAL
    assert "multiples of 256" in _lib.last_error()
    assert lib.pm_gram(FAKE, 256, 256, FAKE, FAKE, ws - 1, None) == _lib.PM_EWORKSPACE
    assert lib.pm_timing_read(None, -1) == _lib.PM_EINVAL
    assert lib.pm_timing_read(None, 0) == 0


def test_ns_form_and_extent_validation(lib):
    assert step(lib, [mat()], hparams(ns_form="gram"), ws_bytes=4096) == _lib.PM_EWORKSPACE  # form accepted
    hp = hparams()
    hp.ns_form = 7
    assert step(lib, [mat()], hp) == _lib.PM_EINVAL
    assert "ns_form" in _lib.last_error()
    with pytest.raises(ValueError, match="ns_form"):
        _lib.ns_form_code("quintic")
    # 256 rows of the padded long side must fit a 32-bit buffer descriptor
    assert step(lib, [mat(rows=256, cols=(1 << 23))]) == _lib.PM_EUNSUPPORTED
    assert "at most" in _lib.last_error()


def test_gemm_symmetric_argument_errors(lib):
    ws = lib.pm_gemm_symmetric_workspace_bytes()
    assert ws > 0
    assert lib.pm_gemm_symmetric(FAKE, FAKE, FAKE, FAKE, 320, 1.0, 0.5, FAKE, ws, None) == _lib.PM_EINVAL
    assert "multiple of 256" in _lib.last_error()
    assert lib.pm_gemm_symmetric(FAKE, FAKE, None, FAKE, 256, 1.0, 0.5, FAKE, ws, None) == _lib.PM_EINVAL
    assert "addend" in _lib.last_error()
    assert lib.pm_gemm_symmetric(None, FAKE, FAKE, FAKE, 256, 1.0, 0.5, FAKE, ws, None) == _lib.PM_EINVAL
    assert lib.pm_gemm_symmetric(FAKE, FAKE, FAKE, FAKE, 256, 1.0, 0.5, FAKE, ws - 1, None) == _lib.PM_EWORKSPACE
    assert lib.pm_gemm_symmetric(FAKE, FAKE, FAKE, FAKE, 256, 1.0, 0.5, FAKE + 8, ws, None) == _lib.PM_EINVAL


def adam_tensor(numel=1000, dts=(0, 0, 0, 0), ptrs=(FAKE,) * 4, step=FAKE, vmax=None):
    t = _lib.PmAdamTensor()
    t.param, t.grad, t.exp_avg, t.exp_avg_sq = ptrs
    t.max_exp_avg_sq = vmax
    t.step = step
    t.numel = numel
    t.param_dtype, t.grad_dtype, t.exp_avg_dtype, t.exp_avg_sq_dtype = dts
    return t


def test_adam_argument_errors(lib):
    def run(ts, ws=FAKE, ws_bytes=1 << 30, **kw):
        hp = _lib.PmAdamHparams(beta1=kw.get("beta1", 0.9), beta2=kw.get("beta2", 0.999), eps=1e-8,
                                weight_decay=kw.get("wd", 0.01), amsgrad=kw.get("amsgrad", 0), maximize=0,
                                decoupled_weight_decay=1)
        a = (_lib.PmAdamTensor * len(ts))(*ts) if ts else None
        return lib.pm_adam_step(a, len(ts), ctypes.byref(hp), None, 1e-3, None, None, ws, ws_bytes, None)

    assert lib.pm_adam_workspace_bytes(-1) == 0
    assert lib.pm_adam_workspace_bytes(3) > 0
    assert run([]) == 0
    assert run([adam_tensor()], beta1=1.0) == _lib.PM_EINVAL
    assert "betas" in _lib.last_error()
    assert run([adam_tensor()], wd=-1.0) == _lib.PM_EINVAL
    assert run([adam_tensor(numel=-1)]) == _lib.PM_EINVAL
    assert run([adam_tensor(step=None)]) == _lib.PM_EINVAL
    assert run([adam_tensor(ptrs=(FAKE, 0, FAKE, FAKE))]) == _lib.PM_EINVAL
    assert run([adam_tensor()], amsgrad=1) == _lib.PM_EINVAL
    assert "max_exp_avg_sq" in _lib.last_error()
    assert run([adam_tensor(dts=(0, 3, 0, 0))]) == _lib.PM_EDTYPE  # f16 (2) is accepted
    assert run([adam_tensor()], ws=0) == _lib.PM_EINVAL
    assert run([adam_tensor()], ws=FAKE + 8) == _lib.PM_EINVAL
    assert run([adam_tensor()], ws_bytes=16) == _lib.PM_EWORKSPACE
    hp = _lib.PmAdamHparams()
    assert lib.pm_adam_step(None, 2, ctypes.byref(hp), None, 1e-3, None, None, FAKE, 1 << 30, None) == _lib.PM_EINVAL
    assert lib.pm_adam_step((_lib.PmAdamTensor * 1)(adam_tensor()), 1, None, None, 1e-3, None, None, FAKE, 1 << 30,
                            None) == _lib.PM_EINVAL


def test_error_text_is_per_thread(lib):
    import threading

    assert step(lib, [mat(pdt=7)]) == _lib.PM_EDTYPE
    seen = []
    t = threading.Thread(target=lambda: seen.append(_lib.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "dtype" in _lib.last_error()


def test_python_check_maps_reference_exception_types(lib):
    assert step(lib, [mat(rows=-3)]) == _lib.PM_EINVAL
    with pytest.raises(ValueError, match="extents"):
        _lib.check(_lib.PM_EINVAL, "muon step")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.PM_EWORKSPACE, "muon step")


def ws_bytes(lib, ms, limit=0):
    hp = hparams(workspace_limit=limit)
    return lib.pm_workspace_bytes(arr(*ms), len(ms), ctypes.byref(hp))


def k_split_partial_bytes(mp, np_):
    """fp32 partial tiles a matrix's K-split stages need: the largest stage's
    tiles x chunks x 256 KiB (the rule of pan2_amd/csrc/pm_tiles.hpp::k_split,
    whose invariants tests/native/tile_order_check.cpp checks)."""
    def k_split(tiles, kt):
        if mp < 512 or kt % 4:
            return 1
        s = 1
        while 2 * s <= 4 and (kt // 4) % (2 * s) == 0 and kt // (2 * s) >= 16 and tiles * 2 * s <= 256:
            s *= 2
        return s
    nt = mp // 256
    sym, full = nt * (nt + 1) // 2, nt * (np_ // 256)
    stages = [(sym, k_split(sym, np_ // 64)), (sym, k_split(sym, mp // 64)), (full, k_split(full, mp // 64))]
    return max([t * s * 256 * 256 * 4 for t, s in stages if s > 1] or [0])


def test_workspace_sizing(lib):
    one = ws_bytes(lib, [mat(1024, 4096)])
    assert one > 0 and one % 256 == 0
    assert ws_bytes(lib, [mat(4096, 1024)]) == one, "a tall matrix is planned as its transpose"
    # bf16 X x2 (ping-pong; no transposed copy) + A + B + the K-split partials
    # (1024 x 4096 splits its gram: 10 tiles x 4 chunks x 256 KiB) dominate
    M, N = 1024, 4096
    kp = k_split_partial_bytes(M, N)
    assert kp == 10 * 4 * 256 * 1024
    assert k_split_partial_bytes(4096, 5120) == 0 and k_split_partial_bytes(256, 4096) == 0
    assert 2 * M * N * 2 + 2 * M * M * 2 + kp <= one <= 2 * M * N * 2 + 2 * M * M * 2 + kp + (1 << 20)
    # padding to 256: 300x700 is planned as 512x768
    assert ws_bytes(lib, [mat(300, 700)]) == ws_bytes(lib, [mat(512, 768)])
    three = ws_bytes(lib, [mat(1024, 4096)] * 3)
    table1 = one - (2 * M * N * 2 + 2 * M * M * 2 + ((M // 64) * (N // 64) * 4 + 255) // 256 * 256 + 256 + kp)
    assert table1 > 0
    assert three > 3 * (one - table1)
    # a cap below the total keeps room for the largest matrix only (groups run in turn)
    capped = ws_bytes(lib, [mat(1024, 4096)] * 3, limit=1)
    assert capped < three and capped >= one
    assert ws_bytes(lib, [mat(pdt=5)]) == 0 and "dtype" in _lib.last_error()


def test_k_split_is_decided_per_call(lib):
    """The K-split depends on the call (pan2_amd/csrc/panmuon.hip::split_call):
    a lone 2048 x 2048 splits every stage and holds the largest stage's partials
    (64 UPDATE tiles x 2 chunks x 256 KiB); 48 of them in one call fill the chip,
    none splits and none holds partials; a workspace cap that groups the call
    does not change that."""
    kp = 64 * 2 * 256 * 1024
    one = ws_bytes(lib, [mat(2048, 2048)])
    many = ws_bytes(lib, [mat(2048, 2048)] * 48)
    assert 48 * (one - kp) - 48 * (1 << 20) <= many <= 48 * (one - kp) + (1 << 20)
    two = ws_bytes(lib, [mat(2048, 2048)] * 2)  # 72 gram tiles: still split 2 ways
    assert 2 * one - (1 << 20) <= two <= 2 * one + (1 << 20)
    capped = ws_bytes(lib, [mat(2048, 2048)] * 48, limit=1)  # groups of one matrix: still unsplit
    assert capped < one - kp + (1 << 20)


def test_k_split_keeps_a_matrix_within_the_noalloc_scratch(lib):
    """A lone 3584 x 6144 splits its grams and symmetric products 2 ways in the
    standard form (105 tiles x 2 chunks x 256 KiB of partials); in the gram
    form (five square buffers) those partials would take it past the
    allocation-free step's 256 MiB scratch, so it stays unsplit there."""
    m, n, kp = 3584, 6144, 105 * 2 * 256 * 1024
    x, sq = m * n * 2, m * m * 2  # X and one square buffer, bf16
    std = ws_bytes(lib, [mat(m, n)])
    assert 2 * x + 2 * sq + kp <= std <= 2 * x + 2 * sq + kp + (1 << 20)
    hp = hparams(ns_form="gram")
    gram = lib.pm_workspace_bytes(arr(mat(m, n)), 1, ctypes.byref(hp))
    assert 2 * x + 5 * sq <= gram <= 2 * x + 5 * sq + (1 << 20) <= _lib.NOALLOC_SCRATCH_BYTES


def test_gram_form_workspace_sizing(lib):
    M, N = 1024, 4096
    std = ws_bytes(lib, [mat(M, N)])
    hp = hparams(ns_form="gram")
    gram = lib.pm_workspace_bytes(arr(mat(M, N)), 1, ctypes.byref(hp))
    # the gram form keeps R, Z, RZ and two Q: three more M x M bf16 matrices
    assert gram - std >= 3 * M * M * 2
    assert gram - std <= 3 * M * M * 2 + (64 << 10)  # plus a larger launch table


def test_ns_workspace_matches_step_workspace(lib):
    m = _lib.PmNsMatrix()
    m.in_, m.out = FAKE, FAKE
    m.rows, m.cols, m.in_ld, m.out_ld, m.in_dtype = 768, 512, 512, 512, 0
    hp = hparams()
    a = (_lib.PmNsMatrix * 1)(m)
    assert lib.pm_ns_workspace_bytes(a, 1, ctypes.byref(hp)) == ws_bytes(lib, [mat(768, 512)])


def test_product_path_has_no_cpu_fallback():
    """pan2_amd never imports the oracle; a CPU tensor is an error, not a fallback."""
    import torch

    for mod in ("pan2_amd._lib", "pan2_amd.optim.patch_muon", "pan2_amd.optim.muon", "pan2_amd.optim.kernels"):
        __import__(mod)
        src = open(sys.modules[mod].__file__).read()
        assert "oracle" not in src, mod
    from pan2_amd.optim.patch_muon import _single_tensor_muon, newton_schulz

    p = torch.zeros(4, 8)
    with pytest.raises(RuntimeError, match="HIP device"):
        _single_tensor_muon([p], [torch.zeros(4, 8)], [torch.zeros(4, 8)], lr=0.1, weight_decay=0.0, momentum=0.9,
                            nesterov=True, ns_coefficients=(3.4445, -4.775, 2.0315), ns_steps=5, eps=1e-7,
                            adjust_lr_fn=None, has_complex=False)
    with pytest.raises(RuntimeError, match="HIP device"):
        newton_schulz(torch.zeros(4, 8), (3.4445, -4.775, 2.0315), 5, 1e-7)
