"""GPU parity of the gram-form Newton–Schulz (PAN 2's production
_gram_newtonschulz_local, pan/optim/patch_muon.py:275-334) and of the
symmetric product that stands in for quack's gemm_symmetric(_out), through
the C ABI.

Tolerances: relative Frobenius error against the fp64 standard quintic (the
two forms are equal in exact arithmetic) <= max(2e-2, 1.25 x the error of the
reference's own algorithm restated in bf16 on the same input). The second term
matters for square matrices only: there the gram form in bf16 is less accurate
(the oracle's bf16 gram form reaches 4.5e-2 on a 512 x 512 Gaussian, where
torch's quintic reaches 1.1e-2), so the gate follows the reference's own
accuracy rather than one it cannot meet. The distance to that bf16
restatement is held to sqrt(2) x that bound (two independent bf16 rounding
sequences, each within the gate of the exact result). The symmetric product is within bf16
rounding of an fp64 product and exactly symmetric; momentum buffers are
bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import muon_ref
from oracle.bf16 import round_bf16
from pan2_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def seeded(shape, seed, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


def rel_fro(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def gram_gate(g, **kw):
    """max(2e-2, 1.25 x the oracle bf16 gram form's error vs the fp64 standard NS)."""
    ref = muon_ref.ns_standard(g, precision="fp64", **kw)
    oracle = muon_ref.ns_gram(g, precision="bf16", **kw)
    return ref, oracle, max(2e-2, 1.25 * rel_fro(oracle, ref))


def sym_bf16(m, seed):
    """A symmetric bf16 matrix with gram-like spectrum (X Xᵀ / ‖X‖²)."""
    x = seeded((m, 2 * m), seed).double().numpy()
    r = x @ x.T / np.sum(x * x)
    return torch.from_numpy(round_bf16(r.astype(np.float32))).to(torch.bfloat16)  # exact: already bf16 values


@pytest.mark.parametrize("m,alpha,beta", [(256, 1.0, 0.0), (512, 2.0315, -4.775), (768, 1.0, 3.4445)])
def test_gemm_symmetric_vs_fp64(m, alpha, beta):
    print(f"gemm_symmetric m={m} alpha={alpha} beta={beta}", flush=True)
    r = sym_bf16(m, 5 + m)
    # z and d are polynomials in r (rounded to bf16), as every operand pair of the gram form is
    rd = r.double().numpy()
    z = torch.from_numpy(round_bf16((2.0315 * rd @ rd - 4.775 * rd).astype(np.float32))).to(torch.bfloat16)
    d = torch.from_numpy(round_bf16((rd @ rd).astype(np.float32))).to(torch.bfloat16) if beta else None
    out = _lib.gemm_symmetric(r.to(DEV), z.to(DEV), d.to(DEV) if d is not None else None, alpha=alpha, beta=beta)
    o = out.float().cpu().numpy().astype(np.float64)
    rf, zf = r.double().numpy(), z.double().numpy()
    ref = alpha * (rf @ zf.T) + (beta * d.double().numpy() if d is not None else 0.0)
    assert np.array_equal(o, round_bf16(o.astype(np.float32))), "output must be bf16 values"
    # the upper triangle is computed and mirrored (diagonal tiles included): exactly symmetric
    assert np.array_equal(o, o.T)
    iu = np.triu_indices(m)
    err = np.abs(o[iu] - ref[iu])
    # bf16 output (half an ulp, 2^-9 relative) plus fp32 accumulation error
    assert np.all(err <= 2.0 ** -8 * np.abs(ref[iu]) + 1e-3 * np.abs(ref).max()), float(err.max())


def test_gemm_symmetric_squares_match_poly_stage():
    """c R R + b R through pm_gemm_symmetric equals the oracle's bf16 rounding of it."""
    m = 512
    r = sym_bf16(m, 77)
    out = _lib.gemm_symmetric(r.to(DEV), r.to(DEV), r.to(DEV), alpha=2.0315, beta=-4.775).float().cpu().numpy()
    rf = r.double().numpy()
    ref = 2.0315 * (rf @ rf) + -4.775 * rf
    assert np.array_equal(out, out.T), "L = R: every tile, diagonal ones included, is exactly symmetric"
    assert rel_fro(out, ref) <= 2.0 ** -8


GRAM_SHAPES = [(1024, 4096), (4096, 1024), (512, 512), (300, 1000), (1000, 300), (64, 96), (513, 257)]


@pytest.mark.parametrize("rows,cols", GRAM_SHAPES)
def test_gram_form_ns_vs_fp64_and_oracle(rows, cols):
    print(f"gram-form ns {rows}x{cols}", flush=True)
    g = seeded((rows, cols), 4321 + rows * 3 + cols)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g.to(DEV), out)], ns_form="gram")
    o = out.float().cpu().numpy()
    ref, oracle, gate = gram_gate(g.numpy())
    assert rel_fro(o, ref) <= gate
    assert rel_fro(o, oracle) <= np.sqrt(2) * gate


@pytest.mark.parametrize("steps", [1, 2, 3, 4, 6])
def test_gram_form_step_counts_and_reset(steps):
    """ns_steps <= 2 has no reset; from 3 on the reset at iteration 2 applies Q and re-grams."""
    print(f"gram-form ns steps={steps}", flush=True)
    g = seeded((512, 1536), 99 + steps)
    out = torch.empty((512, 1536), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g.to(DEV), out)], ns_steps=steps, ns_form="gram")
    o = out.float().cpu().numpy()
    ref, oracle, gate = gram_gate(g.numpy(), ns_steps=steps)
    assert rel_fro(o, ref) <= gate
    assert rel_fro(o, oracle) <= np.sqrt(2) * gate


def test_gram_form_per_step_coefficients():
    coeffs = [(3.4445, -4.7750, 2.0315), (3.0, -3.2, 1.2), (3.4445, -4.7750, 2.0315), (2.5, -2.0, 0.6),
              (1.9, -1.4, 0.5)]
    g = seeded((768, 2048), 2024)
    out = torch.empty((768, 2048), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g.to(DEV), out)], ns_coefficients=coeffs, ns_steps=5, ns_form="gram")
    o = out.float().cpu().numpy()
    ref, oracle, gate = gram_gate(g.numpy(), ns_coefficients=coeffs, ns_steps=5)
    assert rel_fro(o, ref) <= gate


def test_gram_form_grouped_equals_single_and_is_deterministic():
    shapes = [(1024, 3072), (512, 512), (2048, 768), (300, 1000)]
    gs = [seeded(s, 600 + i).to(DEV) for i, s in enumerate(shapes)]
    outs = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(gs, outs)), ns_form="gram")
    again = [torch.empty_like(o) for o in outs]
    _lib.newton_schulz_into(list(zip(gs, again)), ns_form="gram")
    for g, o, a in zip(gs, outs, again):
        single = torch.empty_like(o)
        _lib.newton_schulz_into([(g, single)], ns_form="gram")
        assert torch.equal(o, single)
        assert torch.equal(o, a)
    # several workspace groups (a tiny cap puts each matrix in a group of its own)
    capped = [torch.empty_like(o) for o in outs]
    _lib.newton_schulz_into(list(zip(gs, capped)), ns_form="gram", workspace_limit=1)
    for o, c in zip(outs, capped):
        assert torch.equal(o, c)


def test_gram_form_zero_input():
    g = torch.zeros((512, 1024), device=DEV)
    out = torch.full((512, 1024), 7.0, dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g, out)], ns_form="gram")
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_gram_form_muon_step(pdt):
    """A full Muon step in gram form through the drop-in API: momentum bit-exact,
    the update within the gate of the fp64 standard NS."""
    import pan2_amd.optim.patch_muon as pm

    shapes = [(512, 1536), (1536, 512), (700, 300)]
    lr, wd = 0.02, 0.01
    ps, gs, bs = [], [], []
    for i, s in enumerate(shapes):
        ps.append(seeded(s, 40 + i, 0.02))
        gs.append(seeded(s, 50 + i, 1e-3))
        bs.append(seeded(s, 60 + i, 1e-3))
    params = [p.to(DEV, pdt).clone() for p in ps]
    bufs = [b.to(DEV).clone() for b in bs]
    saved = pm.NS_FORM
    try:
        pm.NS_FORM = "gram"
        pm._single_tensor_muon(params, [g.to(DEV, pdt) for g in gs], bufs, lr=lr, weight_decay=wd,
                               momentum=0.95, nesterov=True, ns_coefficients=(3.4445, -4.7750, 2.0315),
                               ns_steps=5, eps=1e-7, adjust_lr_fn=None, has_complex=False)
    finally:
        pm.NS_FORM = saved
    torch.cuda.synchronize()
    for i, s in enumerate(shapes):
        p0 = ps[i].to(pdt).float().numpy()
        g0 = gs[i].to(pdt).float().numpy()
        ref_p, ref_b, ref_o = muon_ref.muon_step(p0, g0, bs[i].numpy(), lr=lr, weight_decay=wd,
                                                 ns_precision="fp64", ns_form="standard")
        assert np.array_equal(bufs[i].cpu().numpy(), ref_b), "momentum must be bit-exact"
        if pdt == torch.float32:
            ratio = muon_ref.adjust_lr_ratio(None, s)
            o_got = (p0.astype(np.float64) * (1 - lr * wd) - params[i].cpu().numpy().astype(np.float64)) / (lr * ratio)
            u = muon_ref.momentum_nesterov(bs[i].numpy(), g0, 0.95, True)[1]
            assert rel_fro(o_got, ref_o) <= gram_gate(u)[2]
        else:
            # bf16 param: one rounding of p*wdf + O*neg, plus the update's own error band
            ratio = muon_ref.adjust_lr_ratio(None, s)
            wdf, neg = muon_ref.step_factors(lr, wd, ratio)
            ref_p = p0 * wdf + ref_o.astype(np.float32) * neg
            got = params[i].float().cpu().numpy()
            u = muon_ref.momentum_nesterov(bs[i].numpy(), g0, 0.95, True)[1]
            # one bf16 ulp for the rounding of a value the update error may move across a rounding
            # boundary, plus the update error itself (elementwise up to 4x the Frobenius gate)
            ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref_p), 1e-30))) - 7)
            band = ulp + 4 * gram_gate(u)[2] * lr * ratio * np.abs(ref_o).max()
            assert np.all(np.abs(got - ref_p) <= band), float(np.abs(got - ref_p).max())
