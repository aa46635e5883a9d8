"""BASELINE configs 2-5 as full Muon steps on the GPU, at their real sizes.

Each config's parameter set is stepped once through torch.optim.Muon with the
HIP path installed (patch_muon, pan/optim/patch_muon.py:337-339) and a device
lr (the reference's tensor-lr path), under adjust_lr_fn "match_rms_adamw" (the
reference factory's default, pan/optim/muon.py:101) and None (torch's).
State per matrix i, drawn on the GPU from seed 1234 + i: grads bf16 N(0, 1e-3),
momentum fp32 N(0, 1e-3); params fp32 N(0, 0.02) for configs 2-4 (the
reference trains fp32 masters, train.py:573-575) and bf16 N(0, 1e-4) for
config 5, BASELINE's 185 GB throughput state (small, so that the bf16 param
still resolves the update: see below). lr 0.02, weight decay 0.01,
momentum 0.95 Nesterov, 5 quintic steps.

Every matrix's momentum buffer is checked bit-exactly on the device against
momentum_dev, a float32 restatement of the momentum update in torch ops that
test_momentum_dev_matches_the_oracle pins to oracle.muon_ref.momentum_nesterov;
the pre-step buffer is drawn again from its seed. A sample of each config's
matrices is checked further (configs 2-4: every distinct shape; config 5:
every distinct shape and every workspace group of the call, the grouping
model checked against the library's own launch records):
- momentum buffer bit-exact against oracle.muon_ref.momentum_nesterov (CPU);
- the update O the step applied, read back as (p0·(1 - lr·wd) - p1) / adjusted_lr,
  within relative Frobenius error 2e-2 of a float32 Newton–Schulz of the
  same momentum-blended gradient u on the GPU (the north star's gate). For
  bf16 params the read-back carries half a bf16 ulp of p1 / adjusted_lr per
  element; the test bounds that term and subtracts nothing;
- O's singular values inside the closed-form band of the quintic over the
  Marchenko-Pastur support (±0.03), or, for square matrices, under the
  quintic's maximum with the bulk matching the float32 reference's;
- max|Δparam| against the float32 reference step, printed beside the north
  star's 1e-3·lr and beside torch's own bf16 Newton–Schulz on the same u
  (TORCH/optim/_muon.py:31-70, stepped the same way). It is gated at
  max(1e-3·adjusted_lr, 1.25 x torch's): no bf16 NS meets 1e-3·lr at these
  shapes, and under "match_rms_adamw" the raw-lr reading would need
  |ΔO| <= 7e-5, below bf16's resolution of O.
With PM_FULL_STEP_LOG set, every checked matrix appends one JSON line there.
"""
import json
import os
import time

import numpy as np
import pytest
import torch

import torch.optim._muon as torch_muon
from oracle import muon_ref
from pan2_amd import _lib
from pan2_amd.optim.patch_muon import patch_muon
from tests.conftest import TORCH_ZEROPOWER
from tests.test_gpu_full_size import band, ns_fp32, singular_values

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
COEFFS = (3.4445, -4.7750, 2.0315)
LR, WD, MU = 0.02, 0.01, 0.95
S = 5120
BLOCK = [(S, S)] * 8 + [(4 * S, S)] * 2 + [(S, 4 * S)] * 2 + [(S, 6 * S)] * 2 + [(4096, S)]
CONFIGS = {2: [(S, S)] * 48, 3: [(4 * S, S)] * 16 + [(S, 4 * S)] * 16, 4: BLOCK, 5: BLOCK * 24}
QUINTIC_MAX = float(muon_ref.quintic_power(np.linspace(1e-6, 1.0, 200001)).max())  # 1.2024
WORKSPACE_LIMIT = 12 << 30  # the library's default cap


@pytest.fixture
def patched():
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
    patch_muon(ns_form="standard")
    yield
    torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = saved


def workspace_groups(shapes, limit=WORKSPACE_LIMIT):
    """Group index of each matrix in one pm_muon_step call: the library sorts
    by padded long side, then padded short side (both descending), and packs
    matrices in that order into groups whose workspace fits the cap (the
    per-matrix workspace of pan2_amd/csrc/panmuon.hip's make_plan, standard
    form: X twice, A and B, the prologue partials). test_full_config_step
    checks the group sizes this model gives against the library's records."""
    def up(x, m=256):
        return (x + m - 1) // m * m

    plans = []
    for i, (r, c) in enumerate(shapes):
        mp, np_ = up(min(r, c)), up(max(r, c))
        ws = 2 * up(mp * np_ * 2) + 2 * up(mp * mp * 2) + up((mp // 64) * (np_ // 64) * 4) + 256
        plans.append((i, mp, np_, ws))
    order = sorted(plans, key=lambda t: (-t[2], -t[1]))
    group, used, g = {}, 0, 0
    for k, (i, _, _, ws) in enumerate(order):
        table = 4096 + 256 * (k + 1)  # descriptor table, generously
        if used and used + ws + table > limit:
            g, used = g + 1, 0
        group[i] = g
        used += ws
    return group


def samples(config, shapes):
    """Indices checked: the first matrix of each distinct shape, and for config
    5 also the first matrix of each workspace group."""
    pick = {}
    for i, s in enumerate(shapes):
        pick.setdefault(("shape", s), i)
    if config == 5:
        for i, g in sorted(workspace_groups(shapes).items()):
            pick.setdefault(("group", g), i)
    return sorted(set(pick.values()))


def draw(i, s, p_std):
    """Matrix i's initial (param fp32, grad bf16, momentum fp32), drawn on the GPU from seed 1234 + i."""
    gen = torch.Generator(device=DEV).manual_seed(1234 + i)
    p = torch.empty(s, device=DEV).normal_(0.0, p_std, generator=gen)
    g = torch.empty(s, device=DEV).normal_(0.0, 1e-3, generator=gen).to(torch.bfloat16)
    b = torch.empty(s, device=DEV).normal_(0.0, 1e-3, generator=gen)
    return p, g, b


def build(shapes, pdt, p_std):
    params, bufs = [], []
    for i, s in enumerate(shapes):
        p0, g, b = draw(i, s, p_std)
        p = torch.nn.Parameter(p0.to(pdt))
        if p.dtype != torch.bfloat16 and hasattr(p, "grad_dtype"):
            p.grad_dtype = None  # bf16 grads on fp32 masters (torch >= 2.10 asks for this opt-in)
        p.grad = g
        bufs.append(b)
        params.append(p)
    return params, bufs


def momentum_dev(buf, grad, mu=MU):
    """The momentum update in float32 torch ops on the device:
    mu·buf + (1 - mu)·g, (1 - mu) itself computed in float32, each product and
    the sum rounded separately (pan/optim/muon_triton.py:44-47)."""
    mu32 = torch.tensor(mu, dtype=torch.float32, device=buf.device)
    omu32 = torch.tensor(1.0, dtype=torch.float32, device=buf.device) - mu32
    return torch.add(torch.mul(buf, mu32), torch.mul(grad.float(), omu32))


def test_momentum_dev_matches_the_oracle():
    """momentum_dev gives the oracle's bits (muon_ref.momentum_nesterov, fp32
    numpy) on seeded tensors, including values whose products round
    differently with a fused multiply-add."""
    gen = torch.Generator("cpu").manual_seed(5)
    b = torch.randn(257, 131, generator=gen) * 1e-3
    g = (torch.randn(257, 131, generator=gen) * 1e-3).to(torch.bfloat16)
    b[0, :4] = torch.tensor([1.0, -3.0e-38, 6.5e4, 0.0])
    g[0, :4] = torch.tensor([1.0, 3.0e-38, -6.5e4, 0.0]).to(torch.bfloat16)
    want, _ = muon_ref.momentum_nesterov(b.numpy(), g.float().numpy(), MU)
    got = momentum_dev(b.to(DEV), g.to(DEV)).cpu().numpy()
    assert np.array_equal(got, want)


def check_all_momenta(config, shapes, bufs, grads, p_std):
    """Every matrix's stepped momentum buffer against momentum_dev of its
    pre-step buffer, drawn again from its seed (one matrix at a time)."""
    for i, s in enumerate(shapes):
        _, g0, b0 = draw(i, s, p_std)
        assert torch.equal(grads[i], g0), f"config {config} matrix {i}: grad changed"
        want = momentum_dev(b0, g0)
        assert torch.equal(bufs[i], want), f"config {config} matrix {i}: momentum differs from momentum_dev"
        del g0, b0, want


def check_matrix(config, i, shape, p0, g, b0, p1, b1, adjust, pdt):
    """Gates on one matrix; returns its record."""
    ref_b, u = muon_ref.momentum_nesterov(b0.cpu().numpy(), g.float().cpu().numpy(), MU)
    assert np.array_equal(b1.cpu().numpy(), ref_b), f"config {config} matrix {i}: momentum differs from the oracle"
    u_dev = torch.from_numpy(u).to(DEV)
    del ref_b, u
    o_ref = ns_fp32(u_dev)
    ratio = muon_ref.adjust_lr_ratio(adjust, shape)
    adj = LR * ratio
    wdf = 1.0 - LR * WD
    o_got = (p0.double() * wdf - p1.double()) / adj
    err = float((o_got - o_ref.double()).norm() / o_ref.double().norm())
    # read-back resolution: half an ulp of each stored param element, over
    # adjusted_lr, as a relative Frobenius norm
    mant = 8 if pdt == torch.bfloat16 else 24
    half_ulp = torch.ldexp(torch.ones_like(p1, dtype=torch.float64), torch.frexp(p1.double())[1] - mant - 1)
    readout = float(half_ulp.norm() / adj / o_ref.double().norm())
    del half_ulp
    sv = singular_values(o_got.float()).cpu().numpy()
    m, n = shape
    if m != n:
        lo, hi = band(m, n)
        band_ok = bool(lo - 0.03 <= sv.min() and sv.max() <= hi + 0.03)
    else:
        sr = singular_values(o_ref).cpu().numpy()
        lo, hi = 0.0, QUINTIC_MAX
        band_ok = bool(sv.max() <= QUINTIC_MAX + 0.03 and
                       all(abs(np.percentile(sv, q) - np.percentile(sr, q)) <= 0.03 for q in (1, 50, 99)))
    # the float32 reference step (the reference's step_param with O from float32 NS)
    wdf32 = torch.tensor(1.0, device=DEV) - torch.tensor(LR, device=DEV) * WD
    neg32 = -(torch.tensor(LR, device=DEV) * ratio)
    p_ref = p0.float() * wdf32 + o_ref * neg32
    dp = float((p1.float() - p_ref).abs().max())
    o_torch = TORCH_ZEROPOWER(u_dev, COEFFS, 5, 1e-7).float()
    dp_torch = float(((p0.float() * wdf32 + o_torch * neg32).to(pdt).float() - p_ref).abs().max())
    rec = {"config": config, "matrix": i, "shape": list(shape), "adjust_lr_fn": adjust, "param_dtype": str(pdt),
           "rel_fro": err, "readout_rel_bound": readout, "sigma_min": float(sv.min()), "sigma_max": float(sv.max()),
           "band": [lo, hi], "band_ok": band_ok, "max_dp_over_lr": dp / LR, "max_dp_over_adj_lr": dp / adj,
           "torch_bf16_max_dp_over_adj_lr": dp_torch / adj, "north_star_dp_met": dp <= 1e-3 * LR}
    print(f"  [{i}] {shape} rel-Frobenius(O) {err:.4f} (read-back <= {readout:.1e}); sigma [{sv.min():.4f}, "
          f"{sv.max():.4f}] band [{lo:.3f}, {hi:.3f}] {'ok' if band_ok else 'OUT'}; max|dp| = {dp / LR:.2e}·lr = "
          f"{dp / adj:.2e}·adj_lr (torch bf16 NS {dp_torch / adj:.2e}·adj_lr; north star 1e-3·lr "
          f"{'met' if dp <= 1e-3 * LR else 'not met'})", flush=True)
    log = os.environ.get("PM_FULL_STEP_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert err <= 2e-2, rec
    assert band_ok, rec
    assert dp <= max(1e-3 * adj, 1.25 * dp_torch), rec
    return rec


@pytest.mark.timeout(600)
@pytest.mark.parametrize("adjust", ["match_rms_adamw", None])
@pytest.mark.parametrize("config", [2, 3, 4, 5])
def test_full_config_step(patched, config, adjust):
    shapes = CONFIGS[config]
    pdt, p_std = (torch.bfloat16, 1e-4) if config == 5 else (torch.float32, 0.02)
    picks = samples(config, shapes)
    print(f"full step config {config} adjust={adjust}: {len(shapes)} matrices, {pdt}, checking {picks}", flush=True)
    params, bufs = build(shapes, pdt, p_std)
    before = {i: (params[i].detach().clone(), bufs[i].clone()) for i in picks}
    opt = torch.optim.Muon(params, lr=torch.tensor(LR, device=DEV), weight_decay=WD, momentum=MU,
                           adjust_lr_fn=adjust)
    for p, b in zip(params, bufs):
        opt.state[p]["momentum_buffer"] = b
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    _lib.timing_read()
    t0 = time.perf_counter()
    try:
        opt.step()
        torch.cuda.synchronize()
    finally:
        launches = _lib.timing_read()
        _lib.timing_enable(False)
    print(f"  step {1e3 * (time.perf_counter() - t0):.1f} ms (first call, includes setup)", flush=True)
    # the library's grouping: one prologue launch per group, with its matrix count
    lib_sizes = [r["n_matrices"] for r in launches if r["kind"] == "prologue"]
    model = workspace_groups(shapes)
    model_sizes = [sum(1 for g in model.values() if g == k) for k in range(max(model.values()) + 1)]
    print(f"  workspace groups: library {lib_sizes}, model {model_sizes}", flush=True)
    assert lib_sizes == model_sizes, "the test's grouping model disagrees with the library"
    if config == 5:
        assert {model[i] for i in picks} == set(range(len(model_sizes))), "a workspace group is not sampled"
    recs = []
    try:
        check_all_momenta(config, shapes, [opt.state[p]["momentum_buffer"] for p in params],
                          [p.grad for p in params], p_std)
        print(f"  momentum of all {len(shapes)} matrices bit-exact", flush=True)
        for i in picks:
            p0, b0 = before[i]
            recs.append(check_matrix(config, i, shapes[i], p0, params[i].grad, b0, params[i].detach(),
                                     opt.state[params[i]]["momentum_buffer"], adjust, pdt))
    finally:
        del opt, params, bufs, before
        torch.cuda.empty_cache()
    print(f"FULLSTEP config={config} adjust={adjust} checked={len(recs)} "
          f"rel_fro_max={max(r['rel_fro'] for r in recs):.4f} "
          f"dp_over_lr_max={max(r['max_dp_over_lr'] for r in recs):.3e} "
          f"dp_over_adj_lr_max={max(r['max_dp_over_adj_lr'] for r in recs):.3e} "
          f"torch_dp_over_adj_lr_max={max(r['torch_bf16_max_dp_over_adj_lr'] for r in recs):.3e} "
          f"band_ok={all(r['band_ok'] for r in recs)}", flush=True)


def test_step_across_workspace_groups_matches_one_group(patched):
    """MODE_STEP with a small workspace cap runs the call as several groups,
    each reusing the one workspace; params and momentum are bit-identical to
    the same step in one group."""
    import pan2_amd.optim.patch_muon as pm

    shapes = [(1024, 1536), (1536, 1024), (512, 2048), (300, 700), (700, 300), (1024, 1024), (96, 900)]
    results = []
    for limit in (0, 24 << 20):
        params, bufs = build(shapes, torch.float32, 0.02)
        opt = torch.optim.Muon(params, lr=torch.tensor(LR, device=DEV), weight_decay=WD, momentum=MU)
        for p, b in zip(params, bufs):
            opt.state[p]["momentum_buffer"] = b
        saved = pm.WORKSPACE_LIMIT
        pm.WORKSPACE_LIMIT = limit
        try:
            opt.step()
        finally:
            pm.WORKSPACE_LIMIT = saved
        torch.cuda.synchronize()
        results.append(([p.detach().clone() for p in params], [b.clone() for b in bufs]))
    assert len(set(workspace_groups(shapes, 24 << 20).values())) >= 3
    for a, b in zip(results[0][0] + results[0][1], results[1][0] + results[1][1]):
        assert torch.equal(a, b)
