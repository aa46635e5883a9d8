"""BASELINE configs 2, 3 and 5 as full Muon steps in the gram form, on the GPU,
at their real sizes.

The gram form (pan/optim/patch_muon.py:275-334) is what the reference's
patch_muon() installs and what the drop-in runs by default. Each config's
parameter set is stepped once through torch.optim.Muon with a device lr under
"match_rms_adamw", on the state of test_gpu_full_step (seed 1234 + i per
matrix). Every distinct shape is checked against:
- an fp32 standard quintic of the same momentum-blended gradient u on the GPU
  (ns_fp32; the two forms are equal in exact arithmetic);
- gram_ns_peer, the reference's algorithm restated in torch bf16 products on
  the device (each product accumulated in fp32 by the BLAS library and rounded
  to bf16 once with its addend, the upper triangle mirrored, as quack's
  gemm_symmetric does); test_gram_peer_is_the_reference_algorithm pins it to
  oracle.muon_ref.ns_gram.
Gates, as in test_gpu_gram_form: rel-Frobenius(O, fp32 NS) <= max(2e-2,
1.25 x the peer's); singular values inside the band the peer's output shows
(the reference's observed band: 1st, 50th and 99th percentiles within 0.03,
the maximum at most 0.03 above the peer's); max|Δparam| against the fp32
reference step <= max(1e-3·adjusted_lr, 1.25 x the peer's). The momentum
update is the same prologue in both forms and is checked bit-exactly for
every matrix in test_gpu_full_step.
"""
import time

import numpy as np
import pytest
import torch

import torch.optim._muon as torch_muon
from oracle import muon_ref
from pan2_amd.optim.patch_muon import patch_muon
from tests.test_gpu_full_size import ns_fp32, rel_fro, singular_values
from tests.test_gpu_full_step import CONFIGS, COEFFS, DEV, LR, MU, WD, build, draw

pytestmark = pytest.mark.gpu


def _sym(a):
    """The upper triangle of a, mirrored (quack's gemm_symmetric stores the
    upper triangle and mirrors it)."""
    up = torch.triu(a)
    return up + torch.triu(a, diagonal=1).t().contiguous()


def gram_ns_peer(g, coeffs=COEFFS, steps=5, eps=1e-7):
    """pan/optim/patch_muon.py:275-334 in torch bf16 products on the device."""
    a, b, c = coeffs
    reset = {2} if steps > 2 else set()
    x = g.to(torch.bfloat16)
    x = x / x.norm().clamp(min=eps)
    tall = x.shape[0] > x.shape[1]
    if tall:
        x = x.t().contiguous()
    r = _sym(torch.mm(x, x.t().contiguous()))
    q = None
    for i in range(steps):
        if i in reset:
            x = torch.mm(q, x)
            r = _sym(torch.mm(x, x.t().contiguous()))
            q = None
        z = _sym(torch.addmm(r, r, r, beta=b, alpha=c))
        if q is None:
            q = z.clone()
            q.diagonal().add_(a)
        else:
            q = _sym(torch.addmm(q, q, z, beta=a))
        if i < steps - 1 and (i + 1) not in reset:
            rz = _sym(torch.addmm(r, r, z, beta=a))
            r = _sym(torch.addmm(rz, z, rz, beta=a))
    x = torch.mm(q, x)
    return x.t().contiguous() if tall else x


@pytest.mark.parametrize("rows,cols", [(256, 1024), (1024, 256), (300, 700), (512, 512)])
def test_gram_peer_is_the_reference_algorithm(rows, cols):
    """The peer against the oracle's bf16 gram form and the fp64 standard NS:
    the gate test_gpu_gram_form applies to the library."""
    gen = torch.Generator("cpu").manual_seed(rows * 7 + cols)
    g = torch.randn(rows, cols, generator=gen)
    ref = muon_ref.ns_standard(g.numpy(), precision="fp64")
    oracle = muon_ref.ns_gram(g.numpy(), precision="bf16")
    gate = max(2e-2, 1.25 * float(np.linalg.norm(oracle - ref) / np.linalg.norm(ref)))
    peer = gram_ns_peer(g.to(DEV)).double().cpu().numpy()
    e_ref = float(np.linalg.norm(peer - ref) / np.linalg.norm(ref))
    e_orc = float(np.linalg.norm(peer - oracle) / np.linalg.norm(oracle))
    print(f"peer {rows}x{cols}: vs fp64 {e_ref:.4f}, vs oracle bf16 {e_orc:.4f}, gate {gate:.4f}", flush=True)
    assert e_ref <= gate
    assert e_orc <= np.sqrt(2) * gate


def _band_ok(sv, sv_peer):
    return bool(sv.max() <= sv_peer.max() + 0.03 and
                all(abs(np.percentile(sv, q) - np.percentile(sv_peer, q)) <= 0.03 for q in (1, 50, 99)))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("config", [2, 3, 5])
def test_full_config_step_gram_form(config):
    shapes = CONFIGS[config]
    pdt, p_std = (torch.bfloat16, 1e-4) if config == 5 else (torch.float32, 0.02)
    adjust = "match_rms_adamw"
    picks = sorted({s: i for i, s in reversed(list(enumerate(shapes)))}.values())
    print(f"gram-form full step config {config}: {len(shapes)} matrices, {pdt}, checking {picks}", flush=True)
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
    patch_muon(ns_form="gram")
    params, bufs = build(shapes, pdt, p_std)
    before = {i: params[i].detach().clone() for i in picks}
    opt = None
    try:
        opt = torch.optim.Muon(params, lr=torch.tensor(LR, device=DEV), weight_decay=WD, momentum=MU,
                               adjust_lr_fn=adjust)
        for p, b in zip(params, bufs):
            opt.state[p]["momentum_buffer"] = b
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        opt.step()
        torch.cuda.synchronize()
        print(f"  step {1e3 * (time.perf_counter() - t0):.1f} ms (first call, includes setup)", flush=True)
    finally:
        torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = saved
    worst = {}
    try:
        for i in picks:
            shape = shapes[i]
            _, g, b0 = draw(i, shape, p_std)
            _, u = muon_ref.momentum_nesterov(b0.cpu().numpy(), g.float().cpu().numpy(), MU)
            u = torch.from_numpy(u).to(DEV)
            del g, b0
            p0, p1 = before[i], params[i].detach()
            ratio = muon_ref.adjust_lr_ratio(adjust, shape)
            adj = LR * ratio
            o_ref = ns_fp32(u)
            o_peer = gram_ns_peer(u).float()
            o_got = (p0.double() * (1.0 - LR * WD) - p1.double()) / adj
            err, err_peer = rel_fro(o_got, o_ref), rel_fro(o_peer, o_ref)
            sv, sv_peer = singular_values(o_got.float()).cpu().numpy(), singular_values(o_peer).cpu().numpy()
            band_ok = _band_ok(sv, sv_peer)
            wdf32 = torch.tensor(1.0, device=DEV) - torch.tensor(LR, device=DEV) * WD
            neg32 = -(torch.tensor(LR, device=DEV) * ratio)
            p_ref = p0.float() * wdf32 + o_ref * neg32
            dp = float((p1.float() - p_ref).abs().max())
            dp_peer = float(((p0.float() * wdf32 + o_peer * neg32).to(pdt).float() - p_ref).abs().max())
            print(f"  [{i}] {shape} rel-Frobenius(O) {err:.4f} (peer {err_peer:.4f}); sigma [{sv.min():.4f}, "
                  f"{sv.max():.4f}] peer [{sv_peer.min():.4f}, {sv_peer.max():.4f}] {'ok' if band_ok else 'OUT'}; "
                  f"max|dp| {dp / adj:.2e}·adj_lr (peer {dp_peer / adj:.2e}·adj_lr)", flush=True)
            assert err <= max(2e-2, 1.25 * err_peer), (i, shape, err, err_peer)
            assert band_ok, (i, shape, sv.min(), sv.max(), sv_peer.min(), sv_peer.max())
            assert dp <= max(1e-3 * adj, 1.25 * dp_peer), (i, shape, dp / adj, dp_peer / adj)
            worst[shape] = (err, err_peer, dp / adj, dp_peer / adj)
            del u, o_ref, o_peer, o_got, p_ref
    finally:
        del opt, params, bufs, before
        torch.cuda.empty_cache()
    print(f"GRAMSTEP config={config} " + "; ".join(
        f"{s}: rel_fro {v[0]:.4f} (peer {v[1]:.4f}) dp/adj_lr {v[2]:.2e} (peer {v[3]:.2e})" for s, v in worst.items()),
        flush=True)
