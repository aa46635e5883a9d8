"""Pins the CPU oracle (oracle/) against torch, hand-worked values, closed forms,
invariants and the committed golden vectors. CPU only."""
import os

import numpy as np
import pytest
import torch

from oracle import bf16, muon_ref
from tests import pins

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "torch_muon_cpu.npz")


def test_round_bf16_matches_torch():
    pins.check_round_bf16(bf16)


def test_adjust_lr_table():
    pins.check_adjust_lr(muon_ref)


def test_momentum():
    pins.check_momentum(muon_ref)


def test_step_param():
    pins.check_step(muon_ref)


def test_ns_closed_form():
    pins.check_ns_closed_form(muon_ref)


def test_ns_invariants():
    pins.check_ns_invariants(muon_ref)


def test_ns_bf16_vs_torch_stock():
    pins.check_ns_bf16_vs_torch(muon_ref)


def test_ns_gram_equals_standard():
    pins.check_ns_gram(muon_ref)


def test_muon_step_vs_torch_stock():
    pins.check_muon_step_vs_torch(muon_ref)


def test_ns_argument_errors_match_torch():
    """TORCH/optim/_muon.py:46-53: step count and rank checks."""
    with pytest.raises(ValueError, match="less than 100"):
        muon_ref.ns_standard(np.ones((4, 4)), ns_steps=100)
    with pytest.raises(ValueError, match="2D"):
        muon_ref.ns_standard(np.ones(4))


def test_ns_flops_counts():
    """F_ns counts the upper triangle incl. the diagonal for both symmetric GEMMs."""
    f_ns, f_dense = muon_ref.ns_flops(4096, 1024, ns_steps=1)
    M, N = 1024, 4096
    assert f_ns == M * (M + 1) * N + M * M * (M + 1) + 2 * M * M * N
    assert f_dense == 4 * M * M * N + 2 * M ** 3
    assert muon_ref.ns_flops(1024, 4096) == muon_ref.ns_flops(4096, 1024)


def test_closed_form_band_config1():
    """Closed-form output band of config 1 (1024x4096 Gaussian): the quintic maps
    the Marchenko–Pastur support of the normalised input into [0.68, 1.134]."""
    M, N = 1024, 4096
    lo = (1 - np.sqrt(M / N)) / np.sqrt(M)  # normalised singular values of a Gaussian
    hi = (1 + np.sqrt(M / N)) / np.sqrt(M)
    xs = np.linspace(lo, hi, 2001)
    ys = pins.quintic_closed_form(xs)
    assert 0.68 <= ys.min() <= 0.69 and 1.13 <= ys.max() <= 1.14, (ys.min(), ys.max())


# ---------------------------------------------------------------- golden vectors


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(GOLDEN):
        pytest.fail(f"golden fixture missing: {GOLDEN} (tests/golden/make_golden.py writes it)")
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _golden_cases(g, prefix):
    return sorted({k.split("/")[1] for k in g if k.startswith(prefix + "/")})


def test_golden_ns_vs_oracle(golden):
    """torch's stock bf16 NS outputs (written on the CPU by make_golden.py) vs the oracle."""
    cases = _golden_cases(golden, "ns")
    assert len(cases) >= 4
    for c in cases:
        G = golden[f"ns/{c}/in"]
        want = bf16.from_bf16_bits(golden[f"ns/{c}/out_bf16"])
        got = muon_ref.ns_standard(G, precision="bf16")
        assert pins.rel(got, want) < 1.5e-2, (c, pins.rel(got, want))
        assert pins.rel(muon_ref.ns_standard(G, precision="fp64"), want) < 2e-2, c


def test_golden_muon_step_vs_oracle(golden):
    cases = _golden_cases(golden, "step")
    assert len(cases) >= 2
    for c in cases:
        p0, g, b0 = (golden[f"step/{c}/{k}"] for k in ("p0", "g", "b0"))
        lr, wd = float(golden[f"step/{c}/lr"]), float(golden[f"step/{c}/wd"])
        adjust = str(golden[f"step/{c}/adjust"])
        adjust = None if adjust == "None" else adjust
        ref_p, ref_b, ref_o = muon_ref.muon_step(p0, g, b0, lr=lr, weight_decay=wd, adjust_lr_fn=adjust,
                                                 ns_precision="bf16")
        assert np.abs(ref_b - golden[f"step/{c}/b1"]).max() <= 8 * 2.0 ** -24 * np.abs(b0).max(), c
        adj = lr * muon_ref.adjust_lr_ratio(adjust, p0.shape)
        assert np.abs(ref_p - golden[f"step/{c}/p1"]).max() <= 2e-2 * adj, c


def test_golden_matches_current_torch(golden):
    """The fixture still matches this torch's stock CPU NS (guards version skew)."""
    from tests.conftest import TORCH_ZEROPOWER

    for c in _golden_cases(golden, "ns"):
        G = torch.from_numpy(golden[f"ns/{c}/in"])
        got = TORCH_ZEROPOWER(G.clone(), pins.COEFFS, 5, 1e-7).float().numpy()
        want = bf16.from_bf16_bits(golden[f"ns/{c}/out_bf16"])
        assert pins.rel(got, want) < 1e-2, c


def test_adam_vs_torch_cpu():
    from oracle import adamw_ref

    pins.check_adam_vs_torch(adamw_ref)


def test_adam_closed_form():
    from oracle import adamw_ref

    pins.check_adam_closed_form(adamw_ref)


def test_adam_f16_storage_matches_torch():
    from oracle import adamw_ref

    pins.check_adam_store_f16(adamw_ref)
