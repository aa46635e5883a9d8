"""Checks that pin the CPU oracle (imported by the oracle tests and the mutant tests).

Each ``check_*`` takes the oracle module (or a copy with a planted mistake) and
raises AssertionError when the module disagrees with something independent of
its own formulas:
  * torch's implementation of the same operation (the reference's CPU path is
    stock torch.optim.Muon, TORCH/optim/_muon.py),
  * exact values of small cases worked out by hand,
  * the closed form of Newton–Schulz on a matrix with a known SVD,
  * invariants the iteration must keep (transpose, scale, zero, NaN).
tests/test_oracle_mutants.py runs the same checks against planted mistakes to
show that each check can fail.
"""
from __future__ import annotations


import numpy as np
import torch

COEFFS = (3.4445, -4.7750, 2.0315)  # TORCH/optim/_muon.py:24-26


def _torch_modules():
    from tests.conftest import TORCH_SINGLE_TENSOR_MUON, TORCH_ZEROPOWER

    return TORCH_ZEROPOWER, TORCH_SINGLE_TENSOR_MUON


# ------------------------------------------------------------------ bf16


def special_fp32():
    """Values that exercise bf16 rounding: exact ties (odd and even), the
    largest finite values, infinities, NaNs and subnormals."""
    bits = [
        0x3F808000,  # 1 + 2^-8: tie, lower bf16 even -> rounds down
        0x3F818000,  # tie with odd lower bf16 -> rounds up
        0x3F80C000, 0x3F804000, 0x3F807FFF, 0x3F808001,
        0x7F7FFFFF,  # FLT_MAX rounds to +inf
        0x7F7F7FFF, 0x7F800000, 0xFF800000,  # near max, +-inf
        0x7FC00000, 0xFFC00001, 0x7F800001,  # quiet NaNs, signalling NaN
        0x00000001, 0x00008000, 0x00018000, 0x807FFFFF,  # subnormals incl. ties
        0x00000000, 0x80000000,
    ]
    return np.array(bits, dtype=np.uint32).view(np.float32)


def check_round_bf16(bf16mod):
    """round_bf16 == torch's fp32 -> bf16 cast (TORCH/optim/_muon.py:55), bitwise."""
    rng = np.random.default_rng(0)
    x = np.concatenate([special_fp32(), rng.standard_normal(4096).astype(np.float32),
                        (rng.standard_normal(512) * 1e-39).astype(np.float32)])
    got = bf16mod.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), "NaN placement differs from torch"
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32)), "bf16 rounding differs from torch"
    # bit helpers are inverse to each other on bf16 values
    assert np.array_equal(bf16mod.from_bf16_bits(bf16mod.to_bf16_bits(x[~nan]))
                          .view(np.uint32), ref[~nan].view(np.uint32))


# ------------------------------------------------------------------ adjust_lr

ADJUST_MODES = (None, "original", "match_rms_adamw", "unknown_mode")
ADJUST_SHAPES = ((256, 256), (1024, 4096), (4096, 1024), (20480, 5120), (128, 4096), (3, 7), (7, 3))


def check_adjust_lr(ref):
    """Equal to torch.optim._muon._adjust_lr(1.0, mode, shape) over every mode x
    shape class (square, wide, tall, chunk-sized rows)."""
    for mode in ADJUST_MODES:
        for shape in ADJUST_SHAPES:
            want = torch.optim._muon._adjust_lr(1.0, mode, torch.Size(shape))
            got = ref.adjust_lr_ratio(mode, shape)
            assert got == want, (mode, shape, got, want)
    # hand-worked values
    assert ref.adjust_lr_ratio(None, (4096, 1024)) == 2.0
    assert ref.adjust_lr_ratio(None, (1024, 4096)) == 1.0
    assert ref.adjust_lr_ratio("match_rms_adamw", (100, 2500)) == 0.2 * 50.0


# ------------------------------------------------------------------ momentum


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def check_momentum(ref):
    """pan/optim/muon_triton.py:44-48 restated: exact small cases and torch's lerp form."""
    # hand-worked exact cases (all values representable): mu = 0.75
    buf = np.array([2.0, 0.0, -4.0], np.float32)
    g = np.array([4.0, 8.0, 4.0], np.float32)
    nb, u = ref.momentum_nesterov(buf, g, 0.75, True)
    # nb = 0.75*buf + 0.25*g ; u = 0.25*g + 0.75*nb
    assert np.array_equal(nb, np.array([2.5, 2.0, -2.0], np.float32)), nb
    assert np.array_equal(u, np.array([2.875, 3.5, -0.5], np.float32)), u
    nb2, u2 = ref.momentum_nesterov(buf, g, 0.75, False)
    assert np.array_equal(nb2, nb) and np.array_equal(u2, nb), "non-Nesterov update is the new buffer"
    # mu = 0: the buffer becomes the gradient
    nb0, u0 = ref.momentum_nesterov(buf, g, 0.0, True)
    assert np.array_equal(nb0, g) and np.array_equal(u0, g)
    # the input buffer is not modified in place by the oracle
    assert np.array_equal(buf, np.array([2.0, 0.0, -4.0], np.float32))
    # torch's stock form (TORCH/optim/_muon.py:310-311): lerp, within 2 ulp
    rng = np.random.default_rng(1)
    b = (rng.standard_normal(20000) * 1e-3).astype(np.float32)
    gr = (rng.standard_normal(20000) * 1e-3).astype(np.float32)
    tb = torch.from_numpy(b.copy())
    tg = torch.from_numpy(gr)
    tb.lerp_(tg, 1 - 0.95)
    tu = tg.lerp(tb, 0.95)
    nb, u = ref.momentum_nesterov(b, gr, 0.95, True)
    # lerp rounds differently from mu*b + (1-mu)*g; both stay within a few
    # units of 2^-24 of the operand magnitudes (cancellation makes ulps of the
    # result meaningless)
    unit = np.float64(2.0) ** -24
    assert (np.abs(nb - tb.numpy()) / (np.abs(b) + np.abs(gr))).max() <= 4 * unit, "new buffer differs from torch"
    assert (np.abs(u - tu.numpy()) / (np.abs(gr) + np.abs(nb))).max() <= 8 * unit, "update differs from torch"


# ------------------------------------------------------------------ param step


def check_step(ref):
    """pan/optim/muon_triton.py:127-131,188-190 restated: exact cases and torch's mul_/add_ form."""
    # p*(1 - lr*wd) - lr*ratio*u with lr=0.5, wd=0.5, ratio=2: p*0.75 - u
    p = np.array([1.0, -2.0, 4.0], np.float32)
    u = np.array([2.0, 1.0, -0.5], np.float32)
    out = ref.step_param(p, u, 0.5, 0.5, 2.0)
    assert np.array_equal(out, np.array([-1.25, -2.5, 3.5], np.float32)), out
    wdf, neg = ref.step_factors(0.5, 0.5, 2.0)
    assert wdf == np.float32(0.75) and neg == np.float32(-1.0)
    # weight decay uses the raw lr, not the adjusted one (pan/optim/muon_triton.py:189)
    wdf, _ = ref.step_factors(0.02, 0.1, 37.0)
    assert wdf == np.float32(1.0 - 0.02 * 0.1)
    # torch's stock step (TORCH/optim/_muon.py:315-318), within 1 ulp
    rng = np.random.default_rng(2)
    p = (rng.standard_normal(20000) * 0.02).astype(np.float32)
    u = (rng.standard_normal(20000) * 0.01).astype(np.float32)
    lr, wd, ratio = 0.02, 0.01, 12.8
    tp = torch.from_numpy(p.copy())
    tp.mul_(1 - lr * wd)
    tp.add_(torch.from_numpy(u), alpha=-(lr * ratio))
    # torch's add_ may fuse the multiply; bound by the operand magnitudes
    got = ref.step_param(p, u, lr, wd, ratio)
    scale = np.abs(p) + np.abs(u) * lr * ratio
    assert (np.abs(got - tp.numpy()) / scale).max() <= 2 * np.float64(2.0) ** -24


# ------------------------------------------------------------------ Newton–Schulz


def quintic_closed_form(x, coeffs=COEFFS, steps=5):
    """Scalar NS map on one normalised singular value, evaluated in Horner form."""
    x = np.asarray(x, np.float64)
    a, b, c = coeffs
    for _ in range(steps):
        x2 = x * x
        x = x * (a + x2 * (b + c * x2))
    return x


def orthogonal(n, rng):
    q, r = np.linalg.qr(rng.standard_normal((n, n)))
    return q * np.sign(np.diag(r))


def known_svd_case(m, n, seed):
    """(G, expected) with G = U diag(s) V^T and expected = U diag(p^5(s/|s|)) V^T."""
    rng = np.random.default_rng(seed)
    k = min(m, n)
    U = orthogonal(m, rng)[:, :k]
    V = orthogonal(n, rng)[:, :k]
    s = np.geomspace(1e-2, 3.0, k)
    G = (U * s) @ V.T
    x = s / np.linalg.norm(s)
    return G, (U * quintic_closed_form(x)) @ V.T


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def check_ns_closed_form(ref, fn_name="ns_standard"):
    """fp64 NS of a matrix with a known SVD equals the singular-value map."""
    fn = getattr(ref, fn_name)
    for (m, n), seed in (((24, 40), 3), ((40, 24), 4), ((32, 32), 5)):
        G, want = known_svd_case(m, n, seed)
        got = fn(G, precision="fp64")
        assert got.shape == G.shape, (fn_name, got.shape, G.shape)
        assert rel(got, want) < 1e-10, (fn_name, (m, n), rel(got, want))
    # the scalar map itself
    xs = np.array([1e-3, 0.01, 0.3, 0.9, 1.0])
    assert np.allclose(ref.quintic_power(xs), quintic_closed_form(xs), rtol=1e-13, atol=0)


def check_ns_invariants(ref, fn_name="ns_standard"):
    fn = getattr(ref, fn_name)
    rng = np.random.default_rng(7)
    G = rng.standard_normal((24, 56))
    O = fn(G, precision="fp64")
    assert rel(fn(G.T.copy(), precision="fp64"), O.T) < 1e-12, "NS(G^T) must be NS(G)^T"
    assert rel(fn(1e3 * G, precision="fp64"), O) < 1e-12, "NS must be scale invariant"
    assert np.count_nonzero(fn(np.zeros((16, 40)), precision="fp64")) == 0, "zero input -> zero output"
    Gn = G.copy()
    Gn[3, 5] = np.nan
    assert np.isnan(fn(Gn, precision="fp64")).all(), "a NaN input poisons every output"


def check_ns_bf16_vs_torch(ref):
    """The bf16 restatement vs torch's stock bf16 NS on the CPU (TORCH/optim/_muon.py:31-70)."""
    zeropower, _ = _torch_modules()
    for (m, n), seed in (((64, 192), 11), ((192, 64), 12), ((96, 96), 13)):
        g = torch.Generator("cpu").manual_seed(seed)
        G = torch.randn(m, n, generator=g)
        want = zeropower(G.clone(), COEFFS, 5, 1e-7).float().numpy()
        got = ref.ns_standard(G.numpy(), precision="bf16")
        exact = ref.ns_standard(G.numpy(), precision="fp64")
        assert rel(got, want) < 1.5e-2, ((m, n), rel(got, want))
        # both bf16 paths are about equally far from exact arithmetic
        e_t, e_o = rel(want, exact), rel(got, exact)
        assert e_o < 2 * e_t + 1e-3, ((m, n), e_o, e_t)
        assert np.array_equal(got, ref.round_bf16(got)), "bf16 NS output must hold bf16 values"


def check_ns_gram(ref):
    """Gram form (pan/optim/patch_muon.py:275-334) == standard form in exact arithmetic."""
    check_ns_closed_form(ref, "ns_gram")
    rng = np.random.default_rng(9)
    for shape in ((24, 72), (72, 24), (40, 40)):
        G = rng.standard_normal(shape)
        for steps in (1, 2, 3, 5):
            a = ref.ns_gram(G, ns_steps=steps, precision="fp64")
            b = ref.ns_standard(G, ns_steps=steps, precision="fp64")
            assert rel(a, b) < 1e-10, (shape, steps, rel(a, b))


def check_muon_step_vs_torch(ref):
    """One oracle Muon step vs stock torch.optim.Muon on the CPU with a float lr
    (the reference's CPU path, pan/optim/muon.py:126-154)."""
    _, single = _torch_modules()
    import torch.optim._muon as tm

    for adjust, shape in ((None, (64, 160)), ("match_rms_adamw", (160, 64))):
        gen = torch.Generator("cpu").manual_seed(21)
        p0 = torch.randn(*shape, generator=gen) * 0.02
        g = torch.randn(*shape, generator=gen) * 1e-3
        b0 = torch.randn(*shape, generator=gen) * 1e-3
        p = torch.nn.Parameter(p0.clone())
        p.grad = g.clone()
        opt = torch.optim.Muon([p], lr=0.02, weight_decay=0.01, momentum=0.95, adjust_lr_fn=adjust)
        opt.state[p]["momentum_buffer"] = b0.clone()
        saved = tm._single_tensor_muon
        tm._single_tensor_muon = single
        try:
            opt.step()
        finally:
            tm._single_tensor_muon = saved
        ref_p, ref_b, ref_o = ref.muon_step(p0.numpy(), g.numpy(), b0.numpy(), lr=0.02, weight_decay=0.01,
                                            adjust_lr_fn=adjust, ns_precision="bf16")
        tb = opt.state[p]["momentum_buffer"].numpy()
        assert np.abs(ref_b - tb).max() <= 4 * 2.0 ** -24 * np.abs(b0.numpy()).max() * 2
        adj = 0.02 * ref.adjust_lr_ratio(adjust, shape)
        # implied orthogonalised update of torch's step
        o_t = (p0.numpy().astype(np.float64) * (1 - 0.02 * 0.01) - p.detach().numpy()) / adj
        assert rel(ref_o, o_t) < 1.5e-2, (adjust, rel(ref_o, o_t))
        assert np.abs(ref_p - p.detach().numpy()).max() <= 2e-2 * adj, (adjust,)


# ------------------------------------------------------------------ Adam / AdamW

ADAM_CASES = [
    # (decoupled, weight_decay, amsgrad, maximize, betas)
    (True, 0.05, False, False, (0.95, 0.95)),   # PAN 2's AdamW (pan/optim/muon.py:155-164, train.py:240)
    (True, 0.0, False, False, (0.9, 0.999)),
    (False, 0.01, False, False, (0.9, 0.999)),  # Adam: L2 decay folded into the grad
    (True, 0.1, True, False, (0.8, 0.99)),
    (True, 0.01, False, True, (0.3, 0.6)),     # maximize; 1 - beta1 >= 0.5 takes lerp's other branch
]


def _adam_torch_cpu(p0, grads, *, lr, betas, eps, wd, decoupled, amsgrad, maximize):
    """torch's single-tensor Adam / AdamW on the CPU (TORCH/optim/adam.py:347-549)."""
    p = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    cls = torch.optim.AdamW if decoupled else torch.optim.Adam
    opt = cls([p], lr=lr, betas=betas, eps=eps, weight_decay=wd, amsgrad=amsgrad, maximize=maximize,
              foreach=False, fused=False)
    for g in grads:
        p.grad = torch.from_numpy(g.copy())
        opt.step()
    st = opt.state[p]
    vmax = st["max_exp_avg_sq"].numpy() if amsgrad else None
    return p.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy(), vmax, float(st["step"])


def check_adam_vs_torch(ref):
    """Three steps of the oracle against torch's CPU Adam / AdamW: the same
    arithmetic up to torch's vectorised lerp fusing its multiply-add (a few
    fp32 ulps)."""
    rng = np.random.default_rng(5)
    lr, eps = 3e-3, 1e-8
    for decoupled, wd, amsgrad, maximize, betas in ADAM_CASES:
        p0 = rng.standard_normal(997).astype(np.float32)
        grads = [(rng.standard_normal(997) * 10.0 ** rng.uniform(-3, 1)).astype(np.float32) for _ in range(3)]
        tp, tm, tv, tx, tstep = _adam_torch_cpu(p0, grads, lr=lr, betas=betas, eps=eps, wd=wd, decoupled=decoupled,
                                                amsgrad=amsgrad, maximize=maximize)
        p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
        x = np.zeros_like(p0) if amsgrad else None
        step = 0.0
        for g in grads:
            p, m, v, x, step = ref.adam_step(p, g, m, v, step, lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
                                             weight_decay=wd, decoupled=decoupled, amsgrad=amsgrad,
                                             max_exp_avg_sq=x, maximize=maximize)
        case = (decoupled, wd, amsgrad, maximize, betas)
        assert step == tstep, case

        def close(a, b, what):
            # a few ulps of the array's scale: a moment near zero comes from cancelling terms
            assert np.all(np.abs(a - b) <= 2e-6 * np.abs(b) + 1e-6 * np.abs(b).max()), (what, case)

        close(m, tm, "exp_avg")
        close(v, tv, "exp_avg_sq")
        if amsgrad:
            close(x, tx, "max_exp_avg_sq")
        # the update is lr-sized: its fp32 error is a few ulps of lr, plus p's own rounding
        assert np.all(np.abs(p - tp) <= 2e-6 * np.abs(tp) + 2e-6 * lr), case


def check_adam_closed_form(ref):
    """First AdamW step from zero state: the bias corrections cancel the
    moment weights, so p1 = p0 (1 - lr wd) - lr g / (|g| + eps)."""
    rng = np.random.default_rng(9)
    p0 = rng.standard_normal(513).astype(np.float32)
    g = (rng.standard_normal(513) * 1e-2).astype(np.float32)
    lr, wd, eps = 1e-3, 0.05, 1e-8
    p, m, v, _, step = ref.adam_step(p0, g, np.zeros_like(p0), np.zeros_like(p0), 0.0, lr=lr, beta1=0.95, beta2=0.95,
                                     eps=eps, weight_decay=wd)
    assert step == 1.0
    g64 = g.astype(np.float64)
    want = p0.astype(np.float64) * (1 - lr * wd) - lr * g64 / (np.abs(g64) + eps)
    assert np.all(np.abs(p - want) <= 4e-7 * np.abs(want) + 1e-6 * lr), float(np.abs(p - want).max())
    np.testing.assert_allclose(m, 0.05 * g64, rtol=1e-6)
    np.testing.assert_allclose(v, 0.05 * g64 * g64, rtol=1e-6)
    # zero grad and no decay: nothing moves
    p2, *_ = ref.adam_step(p0, np.zeros_like(p0), np.zeros_like(p0), np.zeros_like(p0), 0.0, lr=lr, beta1=0.9,
                           beta2=0.999, eps=eps, weight_decay=0.0)
    assert np.array_equal(p2, p0)


def check_adam_store_f16(ref):
    """The oracle's fp16 storage rounding equals torch's own float32 -> float16
    cast (round to nearest even) bit for bit: random values over fp16's range,
    exact ties, overflow to inf, subnormals and NaN."""
    import torch

    rng = np.random.default_rng(11)
    x = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-9, 4.9, 20000)).astype(np.float32)
    one = np.float32(1.0)
    ties = np.array([one + np.float32(2.0 ** -11), one + np.float32(3 * 2.0 ** -11), 65520.0, -65520.0, 2.0 ** -25,
                     3 * 2.0 ** -25, 1e-8, 7e4, np.nan, np.inf, -0.0], dtype=np.float32)
    x = np.concatenate([x, ties])
    with np.errstate(over="ignore"):
        got = ref._store(x, "f16")
    want = torch.from_numpy(x).half().float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)  # NaN payloads are not compared
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
