"""Parity at BASELINE's full sizes, through properties that do not depend on size.

Every distinct matrix shape of configs 1-5 (and one of PAN 2's chunked QKV
weights) goes through pm_newton_schulz on a seeded Gaussian input and is checked
against:
- a float32 restatement of the standard quintic on the GPU (torch matmuls in
  fp32; the north star's rel-Frobenius gate 2e-2 is defined against fp32 NS),
- the closed form of the iteration on the input's singular values: NS maps each
  normalised singular value x to p⁵(x), p(x) = a·x + b·x³ + c·x⁵
  (oracle.muon_ref.quintic_power), so the output's singular values lie in
  p⁵ of the Marchenko-Pastur support of the normalised Gaussian,
  [(1 - √c)/√M, (1 + √c)/√M] with c = M/N, widened by 0.03 for bf16 rounding.
  Square matrices reach down to 0 there; for them the top of the band (the
  quintic's maximum, 1.2024) and the bulk (1st-99th percentile against the
  fp32 reference's, ±0.03) are checked instead.
"""
import math

import numpy as np
import pytest
import torch

from oracle import muon_ref
from pan2_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
COEFFS = (3.4445, -4.7750, 2.0315)
S = 5120
SHAPES = [(1024, 4096), (S, S), (4 * S, S), (S, 4 * S), (S, 6 * S), (4096, S)]


def gaussian(shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32)


def ns_fp32(g):
    """Standard quintic (TORCH/optim/_muon.py:55-69) in float32 on the GPU."""
    x = g.float()
    tall = x.shape[-2] > x.shape[-1]
    if tall:
        x = x.mT.contiguous()
    x = x / x.norm(dim=(-2, -1), keepdim=True).clamp(min=1e-7)
    a, b, c = COEFFS
    for _ in range(5):
        A = x @ x.mT.contiguous()
        B = b * A + c * (A @ A)
        x = a * x + B @ x
    return x.mT.contiguous() if tall else x


def test_ns_fp32_matches_the_fp64_oracle():
    """ns_fp32, the float32 reference the full-size and full-step tests gate
    against, agrees with the oracle's float64 standard quintic
    (muon_ref.ns_standard, pinned by tests/pins.py) on a wide and a tall
    matrix, to float32 rounding; a dropped term, a transposed operand or a
    missing normalisation would be off by O(1)."""
    for shape in ((64, 96), (96, 64)):
        gen = torch.Generator("cpu").manual_seed(7)
        x = torch.randn(*shape, generator=gen, dtype=torch.float64)
        want = muon_ref.ns_standard(x.numpy(), COEFFS, 5, 1e-7, precision="fp64")
        got = ns_fp32(x.float().to(DEV)).double().cpu().numpy()
        rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
        assert got.shape == want.shape and rel < 1e-5, (shape, rel)


def singular_values(o):
    """Singular values of o (short side), from the eigenvalues of its float32 gram
    (absolute error ~1e-6 on σ², far inside the 0.03 slack)."""
    o = o.float()
    gram = o @ o.mT.contiguous() if o.shape[-2] <= o.shape[-1] else o.mT.contiguous() @ o
    return torch.linalg.eigvalsh(gram).clamp(min=0).sqrt()


def band(m, n):
    """p⁵ over the Marchenko-Pastur support of an m x n Gaussian normalised by its Frobenius norm."""
    M, N = min(m, n), max(m, n)
    c = M / N
    lo, hi = (1 - math.sqrt(c)) / math.sqrt(M), (1 + math.sqrt(c)) / math.sqrt(M)
    y = muon_ref.quintic_power(np.linspace(lo, hi, 20001))
    return float(y.min()), float(y.max())


def rel_fro(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_full_size_ns(rows, cols):
    print(f"full-size ns {rows}x{cols}", flush=True)
    g = gaussian((rows, cols), rows + 7 * cols)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g, out)])
    ref = ns_fp32(g)
    err = rel_fro(out.float(), ref)
    s = singular_values(out.float()).cpu().numpy()
    print(f"  rel-Frobenius vs fp32 {err:.4f}; singular values [{s.min():.4f}, {s.max():.4f}]", flush=True)
    assert err <= 2e-2
    if rows != cols:
        lo, hi = band(rows, cols)
        assert lo - 0.03 <= s.min() and s.max() <= hi + 0.03, (s.min(), s.max(), lo, hi)
    else:
        top = float(muon_ref.quintic_power(np.linspace(1e-6, 1.0, 200001)).max())  # 1.2024
        assert s.max() <= top + 0.03
        sr = singular_values(ref).cpu().numpy()
        for q in (1, 50, 99):
            assert abs(np.percentile(s, q) - np.percentile(sr, q)) <= 0.03, q


def test_full_size_chunked_qkv_weight():
    """One of PAN 2's QKV weights (24576 x 4096) as its 192 row blocks of 128 x 4096."""
    g = gaussian((192, 128, 4096), 4242)
    out = torch.empty_like(g, dtype=torch.bfloat16)
    _lib.newton_schulz_into([(g[i], out[i]) for i in range(192)])
    ref = ns_fp32(g)
    lo, hi = band(128, 4096)
    for i in range(192):
        assert rel_fro(out[i].float(), ref[i]) <= 2e-2, i
    s = singular_values(out.float()).cpu().numpy()
    assert lo - 0.03 <= s.min() and s.max() <= hi + 0.03, (s.min(), s.max(), lo, hi)


@pytest.mark.parametrize("rows,cols", [(128, 1 << 22), ((1 << 22) + 256, 100), (256, 1 << 21)])
def test_long_side_near_the_offset_limits(rows, cols):
    """Long sides of millions of elements: the 32-bit buffer offsets of the
    small-matrix kernels (128 rows of X) and of the engine's 256-row panels stay
    inside their ranges; the result keeps the fp32 gate and the band."""
    print(f"long-side ns {rows}x{cols}", flush=True)
    g = gaussian((rows, cols), 99 + rows + cols)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g, out)])
    ref = ns_fp32(g)
    err = rel_fro(out.float(), ref)
    s = singular_values(out.float()).cpu().numpy()
    lo, hi = band(rows, cols)
    print(f"  rel-Frobenius vs fp32 {err:.4f}; singular values [{s.min():.4f}, {s.max():.4f}] in [{lo:.4f}, {hi:.4f}]",
          flush=True)
    assert err <= 2e-2
    assert lo - 0.03 <= s.min() and s.max() <= hi + 0.03
