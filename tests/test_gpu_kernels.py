"""GPU parity of libpanmuon's kernels against the CPU oracle (C ABI via ctypes).

Tolerances (north star): NS relative Frobenius error <= 2e-2 against the fp64
restatement of torch's quintic; elementwise momentum/step are bit-exact against
the oracle's fp32 arithmetic; the symmetric gram is within bf16 rounding of an
fp64 product and exactly symmetric.
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
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std)


def rel_fro(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("rows,cols", [(256, 256), (512, 1024), (1024, 4096), (768, 512)])
def test_gram_symmetric_vs_fp64(rows, cols):
    print(f"gram {rows}x{cols}", flush=True)
    x = seeded((rows, cols), 11 + rows).to(torch.bfloat16)
    c = _lib.gram(x.to(DEV)).float().cpu().numpy()
    torch.cuda.synchronize()
    xf = x.float().numpy().astype(np.float64)
    ref = xf @ xf.T
    assert np.array_equal(c, c.T), "mirrored tiles must make the gram exactly symmetric"
    # bf16 output: at most half an ulp (2^-9 relative) plus fp32 accumulation error
    err = np.abs(c - ref)
    assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-3 * np.abs(ref).max()), float(err.max())
    assert np.array_equal(c, round_bf16(c)), "output must be bf16 values"


def test_gram_rejects_unpadded_shapes():
    x = torch.zeros((256, 320), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="multiples of 256"):
        _lib.gram(x)


NS_SHAPES = [(256, 256), (1024, 4096), (4096, 1024), (300, 700), (700, 300), (64, 96), (513, 257)]


@pytest.mark.parametrize("rows,cols", NS_SHAPES)
def test_newton_schulz_vs_fp64(rows, cols):
    print(f"ns {rows}x{cols}", flush=True)
    g = seeded((rows, cols), 1234 + rows * 7 + cols)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(g.to(DEV), out)])
    o = out.float().cpu().numpy()
    ref = muon_ref.ns_standard(g.numpy(), precision="fp64")
    err = rel_fro(o, ref)
    assert err <= 2e-2, err
    # and close to the oracle's bf16 restatement of torch's rounding points
    assert rel_fro(o, muon_ref.ns_standard(g.numpy(), precision="bf16")) <= 2e-2


def test_newton_schulz_bf16_input_and_band(torch_stock_muon):
    """Config 1 shape: singular values inside the band torch's own bf16 NS shows."""
    from tests.conftest import TORCH_ZEROPOWER

    g = seeded((1024, 4096), 1234)
    gb = g.to(torch.bfloat16).to(DEV)
    out = torch.empty((1024, 4096), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(gb, out)])
    ref_t = TORCH_ZEROPOWER(gb.clone(), (3.4445, -4.7750, 2.0315), 5, 1e-7)
    s = torch.linalg.svdvals(out.float()).cpu().numpy()
    st = torch.linalg.svdvals(ref_t.float()).cpu().numpy()
    lo, hi = st.min(), st.max()
    slack = 0.02
    assert s.min() >= lo - slack and s.max() <= hi + slack, (s.min(), s.max(), lo, hi)
    # closed-form band of the quintic over the Marchenko–Pastur support
    assert 0.68 - slack <= s.min() and s.max() <= 1.134 + slack
    assert rel_fro(out.float().cpu().numpy(), ref_t.float().cpu().numpy()) <= 2e-2


def test_grouped_call_equals_single_calls():
    shapes = [(256, 512), (512, 256), (300, 700), (1024, 256), (256, 256)]
    ins = [seeded(s, 50 + i).to(DEV) for i, s in enumerate(shapes)]
    grouped = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(ins, grouped)))
    for x, gout in zip(ins, grouped):
        single = torch.empty_like(gout)
        _lib.newton_schulz_into([(x, single)])
        assert torch.equal(single, gout)


def test_workspace_groups_equal_one_group():
    """A small workspace cap forces several groups; results must not change."""
    shapes = [(512, 512), (256, 768), (768, 256)]
    ins = [seeded(s, 70 + i).to(DEV) for i, s in enumerate(shapes)]
    a = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    b = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(ins, a)))
    _lib.newton_schulz_into(list(zip(ins, b)), workspace_limit=1)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_deterministic():
    x = seeded((512, 1024), 99).to(DEV)
    o1 = torch.empty((512, 1024), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    _lib.newton_schulz_into([(x, o1)])
    _lib.newton_schulz_into([(x, o2)])
    assert torch.equal(o1, o2)


def test_zero_and_nan_inputs():
    z = torch.zeros((256, 512), device=DEV)
    o = torch.empty((256, 512), dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(z, o)])
    assert torch.count_nonzero(o.float()) == 0
    x = seeded((256, 512), 3)
    x[17, 33] = float("nan")
    _lib.newton_schulz_into([(x.to(DEV), o)])
    assert torch.isnan(o.float()).all()


@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nesterov", [True, False])
def test_momentum_bit_exact(gdt, nesterov):
    n = 1 << 16
    g = seeded((n,), 5, 1e-3).to(gdt)
    b = seeded((n,), 6, 1e-3)
    bd, gd = b.to(DEV), g.to(DEV)
    u = torch.empty(n, dtype=torch.float32, device=DEV)
    _lib.momentum_nesterov_into(bd, gd, u, 0.95, nesterov=nesterov)
    nb, uref = muon_ref.momentum_nesterov(b.numpy(), g.float().numpy(), 0.95, nesterov)
    assert np.array_equal(bd.cpu().numpy(), nb)
    assert np.array_equal(u.cpu().numpy(), uref)


@pytest.mark.parametrize("lr_kind", ["float", "device", "cpu_tensor"])
def test_step_param_bit_exact(lr_kind):
    n = 1 << 16
    p = seeded((n,), 8, 0.02)
    u = seeded((n,), 9, 0.01).to(torch.bfloat16)
    pd = p.to(DEV)
    lr = 0.02
    lr_arg = {"float": lr, "device": torch.tensor(lr, device=DEV),
              "cpu_tensor": torch.tensor(lr)}[lr_kind]
    _lib.step_param_inplace(pd, u.to(DEV), lr_arg, 0.01, 1.5)
    if lr_kind == "device":
        lr32 = np.float32(lr)
        wdf = np.float32(1.0) - lr32 * np.float32(0.01)
        neg = -(lr32 * np.float32(1.5))
        ref = (p.numpy() * wdf).astype(np.float32) + (u.float().numpy() * neg).astype(np.float32)
    else:
        lr_used = float(torch.tensor(lr).item()) if lr_kind == "cpu_tensor" else lr
        ref = muon_ref.step_param(p.numpy(), u.float().numpy(), lr_used, 0.01, 1.5)
    assert np.array_equal(pd.cpu().numpy(), ref)


def test_newton_schulz_vs_golden_torch_outputs():
    """HIP NS on the committed golden inputs vs torch's stock bf16 NS outputs
    (tests/golden/torch_muon_cpu.npz, written on the CPU by make_golden.py)."""
    import os

    from oracle.bf16 import from_bf16_bits

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "torch_muon_cpu.npz")
    with np.load(path, allow_pickle=False) as z:
        cases = sorted({k.split("/")[1] for k in z.files if k.startswith("ns/")})
        assert cases
        for c in cases:
            G = z[f"ns/{c}/in"]
            want = from_bf16_bits(z[f"ns/{c}/out_bf16"])
            out = torch.empty(G.shape, dtype=torch.bfloat16, device=DEV)
            _lib.newton_schulz_into([(torch.from_numpy(G).to(DEV), out)])
            got = out.float().cpu().numpy()
            exact = muon_ref.ns_standard(G, precision="fp64")
            # the gate is against exact arithmetic; torch's bf16 output is itself
            # up to 2e-2 from it, so two conforming results differ by <= 4e-2
            assert rel_fro(got, exact) <= 2e-2, (c, rel_fro(got, exact))
            assert rel_fro(want, exact) <= 2e-2, (c, "torch bf16", rel_fro(want, exact))
            assert rel_fro(got, want) <= 4e-2, (c, rel_fro(got, want))
