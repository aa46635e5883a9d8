"""GPU parity of a full Muon step through the drop-in torch.optim.Muon API.

Gates (north star): the orthogonalised update is within relative Frobenius
error 2e-2 of the fp64 restatement of torch's NS; momentum buffers are
bit-exact against the oracle; max |Δparam| against the fp32 reference step is
<= 1e-3·lr, or, where torch's own bf16 Newton–Schulz on the same input already
exceeds that bound, no more than 1.25x torch's own max |Δparam| (measured in
the test). On the config-1 shape torch's bf16 path lands at ~1.44e-3·lr: the
elementwise spread of any bf16 NS there is larger than 1e-3·lr.
"""
import json
import os

import numpy as np
import pytest
import torch

import torch.optim._muon as torch_muon
from oracle import muon_ref
from pan2_amd import _lib
from pan2_amd.optim.muon import build_native_muon_optimizers
from pan2_amd.optim.patch_muon import patch_muon
from tests.test_gpu_full_size import band

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture
def patched():
    """The HIP path with the standard quintic, whose gates these tests check
    (the gram form, the drop-in's default, has its own in test_gpu_gram_form)."""
    import pan2_amd.optim.patch_muon as pm

    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, pm.NS_FORM)
    patch_muon(ns_form="standard")
    yield
    torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, pm.NS_FORM = saved


def cpu_rand(shape, seed, std):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


def run_step(shapes, *, lr, wd=0.01, adjust=None, pdt=torch.float32, gdt=torch.float32, mdt=torch.float32,
             seed=1234, lr_kind="device"):
    params, init = [], []
    for i, s in enumerate(shapes):
        p0 = cpu_rand(s, seed + 3 * i, 0.02)
        g = cpu_rand(s, seed + 3 * i + 1, 1e-3)
        b = cpu_rand(s, seed + 3 * i + 2, 1e-3)
        p = torch.nn.Parameter(p0.to(pdt).to(DEV))
        p.grad = g.to(gdt).to(DEV)
        params.append(p)
        init.append((p0.to(pdt).float().numpy(), g.to(gdt).float().numpy(), b.to(mdt).float().numpy()))
    lr_arg = torch.tensor(lr, device=DEV) if lr_kind == "device" else lr
    opt = torch.optim.Muon(params, lr=lr_arg, weight_decay=wd, momentum=0.95, adjust_lr_fn=adjust)
    for p, (_, _, b) in zip(params, init):
        opt.state[p]["momentum_buffer"] = torch.from_numpy(b).to(mdt).to(DEV)
    opt.step()
    torch.cuda.synchronize()
    return params, opt, init


@pytest.mark.parametrize("adjust", [None, "match_rms_adamw"])
def test_step_config1_gate(patched, adjust):
    """Config-1 shape, fp32 state, against the fp32 reference step."""
    from tests.conftest import TORCH_ZEROPOWER

    lr = 0.02
    shape = (1024, 4096)
    print(f"step gate {shape} adjust={adjust}", flush=True)
    params, opt, init = run_step([shape], lr=lr, adjust=adjust)
    p0, g, b = init[0]
    ref_p, ref_b, ref_o = muon_ref.muon_step(p0, g, b, lr=lr, weight_decay=0.01, adjust_lr_fn=adjust,
                                             ns_precision="fp32")
    got_p = params[0].detach().cpu().numpy()
    assert np.array_equal(opt.state[params[0]]["momentum_buffer"].cpu().numpy(), ref_b)
    ratio = muon_ref.adjust_lr_ratio(adjust, shape)
    dp = float(np.abs(got_p - ref_p).max())
    o_got = (p0.astype(np.float64) * (1 - lr * 0.01) - got_p) / (lr * ratio)
    err = float(np.linalg.norm(o_got - ref_o) / np.linalg.norm(ref_o))
    # torch's own bf16 NS (the reference's PyTorch path) on the same update, on the GPU
    _, u = muon_ref.momentum_nesterov(b, g, 0.95)
    o_t = TORCH_ZEROPOWER(torch.from_numpy(u).to(DEV), (3.4445, -4.7750, 2.0315), 5, 1e-7).float().cpu().numpy()
    dp_torch = float(np.abs(muon_ref.step_param(p0, o_t, lr, 0.01, ratio) - ref_p).max())
    sv = np.linalg.svd(o_got, compute_uv=False)
    lo, hi = band(*shape)  # closed-form band: the quintic over the Marchenko-Pastur support
    band_ok = bool(lo - 0.03 <= sv.min() and sv.max() <= hi + 0.03)
    print(f"  rel-Frobenius(O)={err:.3e} max|dp|/adj_lr={dp / (lr * ratio):.3e} "
          f"torch-bf16 max|dp|/adj_lr={dp_torch / (lr * ratio):.3e} sigma [{sv.min():.4f}, {sv.max():.4f}]")
    log = os.environ.get("PM_FULL_STEP_LOG")
    if log:  # the same record as tests/test_gpu_full_step.py writes for configs 2-5
        with open(log, "a") as f:
            f.write(json.dumps({"config": 1, "matrix": 0, "shape": list(shape), "adjust_lr_fn": adjust,
                                "param_dtype": "torch.float32", "rel_fro": err, "readout_rel_bound": 0.0,
                                "sigma_min": float(sv.min()), "sigma_max": float(sv.max()), "band": [lo, hi],
                                "band_ok": band_ok, "max_dp_over_lr": dp / lr, "max_dp_over_adj_lr": dp / (lr * ratio),
                                "torch_bf16_max_dp_over_adj_lr": dp_torch / (lr * ratio),
                                "north_star_dp_met": dp <= 1e-3 * lr}) + "\n")
    assert err <= 2e-2
    assert band_ok
    assert dp <= max(1e-3 * lr * ratio, 1.25 * dp_torch)


@pytest.mark.parametrize("lr_kind", ["device", "float"])
def test_step_mixed_shapes(patched, lr_kind):
    shapes = [(256, 512), (512, 256), (300, 700), (700, 300), (256, 256), (96, 64)]
    lr = 0.02
    params, opt, init = run_step(shapes, lr=lr, lr_kind=lr_kind)
    for p, (p0, g, b), s in zip(params, init, shapes):
        _, ref_b, ref_o = muon_ref.muon_step(p0, g, b, lr=lr, weight_decay=0.01, ns_precision="fp64")
        ratio = muon_ref.adjust_lr_ratio(None, s)
        o_got = (p0.astype(np.float64) * (1 - lr * 0.01) - p.detach().cpu().numpy()) / (lr * ratio)
        err = float(np.linalg.norm(o_got - ref_o) / np.linalg.norm(ref_o))
        assert err <= 2e-2, (s, err)
        assert np.array_equal(opt.state[p]["momentum_buffer"].cpu().numpy(), ref_b)


def test_step_bf16_state(patched):
    """bf16 params and grads with fp32 momentum (the BASELINE throughput dtypes)."""
    shapes = [(512, 1024), (1024, 512)]
    lr = 0.02
    params, opt, init = run_step(shapes, lr=lr, pdt=torch.bfloat16, gdt=torch.bfloat16)
    for p, (p0, g, b), s in zip(params, init, shapes):
        _, ref_b, ref_o = muon_ref.muon_step(p0, g, b, lr=lr, weight_decay=0.01, ns_precision="fp64")
        assert np.array_equal(opt.state[p]["momentum_buffer"].cpu().numpy(), ref_b)
        ratio = muon_ref.adjust_lr_ratio(None, s)
        wdf, neg = muon_ref.step_factors(lr, 0.01, ratio)
        # bf16 param: one rounding of p*wdf + O*neg; compare against that band
        ref_p = p0 * wdf + ref_o.astype(np.float32) * neg
        got = p.detach().float().cpu().numpy()
        ulp = np.abs(ref_p) * 2.0 ** -8
        assert np.all(np.abs(got - ref_p) <= ulp + 2e-2 * lr * ratio * np.abs(ref_o).max()), float(
            np.abs(got - ref_p).max())


def test_grad_none_skipped_and_zero_grad(patched):
    a = torch.nn.Parameter(cpu_rand((256, 256), 1, 0.02).to(DEV))
    b = torch.nn.Parameter(cpu_rand((256, 256), 2, 0.02).to(DEV))
    a0, b0 = a.detach().clone(), b.detach().clone()
    a.grad = torch.zeros_like(a)
    opt = torch.optim.Muon([a, b], lr=torch.tensor(0.02, device=DEV), weight_decay=0.01)
    opt.step()
    torch.cuda.synchronize()
    assert torch.equal(b.detach(), b0), "param without grad must not change"
    assert b not in opt.state or "momentum_buffer" not in opt.state[b]
    # zero grad: zero update, only the decoupled weight decay applies
    wdf = np.float32(1.0) - np.float32(0.02) * np.float32(0.01)
    assert torch.equal(a.detach().cpu(), (a0.cpu() * torch.tensor(wdf)))


def test_empty_param_is_left_alone(patched):
    """An empty 2-D param steps as in torch (TORCH/optim/_muon.py:31-70 and
    :290-320 leave it as it is): no error, the other params of the group
    step as they would without it, and the NS of an empty matrix is empty."""
    a = torch.nn.Parameter(cpu_rand((256, 512), 5, 0.02).to(DEV))
    e = torch.nn.Parameter(torch.zeros((0, 128), device=DEV))
    twin = torch.nn.Parameter(a.detach().clone())
    for p in (a, twin):
        p.grad = cpu_rand((256, 512), 6, 1e-3).to(DEV)
    e.grad = torch.zeros_like(e)
    torch.optim.Muon([a, e], lr=torch.tensor(0.02, device=DEV), weight_decay=0.01).step()
    torch.optim.Muon([twin], lr=torch.tensor(0.02, device=DEV), weight_decay=0.01).step()
    torch.cuda.synchronize()
    assert e.shape == (0, 128)
    assert torch.equal(a.detach(), twin.detach())
    out = torch_muon._zeropower_via_newtonschulz(torch.zeros((0, 64), device=DEV), (3.4445, -4.7750, 2.0315), 5, 1e-7)
    assert out.shape == (0, 64) and out.dtype == torch.bfloat16


def test_nan_grad_propagates(patched):
    p = torch.nn.Parameter(cpu_rand((256, 512), 4, 0.02).to(DEV))
    g = cpu_rand((256, 512), 5, 1e-3)
    g[3, 7] = float("nan")
    p.grad = g.to(DEV)
    opt = torch.optim.Muon([p], lr=torch.tensor(0.02, device=DEV))
    opt.step()
    torch.cuda.synchronize()
    assert torch.isnan(p.detach()).all()


def test_chunked_param_group(patched):
    """adjust_lr_fn tuple (base, 0, n): row blocks orthogonalised independently,
    lr adjusted with the chunk shape (pan/optim/patch_muon.py:63-68,142)."""
    shape, n = (512, 768), 2
    lr = 0.02
    p0 = cpu_rand(shape, 9, 0.02)
    g = cpu_rand(shape, 10, 1e-3)
    p = torch.nn.Parameter(p0.to(DEV))
    p.grad = g.to(DEV)
    opt = torch.optim.Muon([{"params": [p], "adjust_lr_fn": ("match_rms_adamw", 0, n)}],
                           lr=torch.tensor(lr, device=DEV), weight_decay=0.01, adjust_lr_fn="match_rms_adamw")
    opt.step()
    torch.cuda.synchronize()
    got = p.detach().cpu().numpy().astype(np.float64)
    rows = shape[0] // n
    ratio = muon_ref.adjust_lr_ratio("match_rms_adamw", (rows, shape[1]))
    for k in range(n):
        sl = slice(k * rows, (k + 1) * rows)
        _, _, ref_o = muon_ref.muon_step(p0.numpy()[sl], g.numpy()[sl], np.zeros((rows, shape[1]), np.float32),
                                         lr=lr, weight_decay=0.01, ns_precision="fp64")
        o_got = (p0.numpy()[sl].astype(np.float64) * (1 - lr * 0.01) - got[sl]) / (lr * ratio)
        assert np.linalg.norm(o_got - ref_o) / np.linalg.norm(ref_o) <= 2e-2


def test_factory_tensor_lr_installs_hip_path():
    model = torch.nn.Sequential(torch.nn.Linear(256, 512, bias=True), torch.nn.Linear(512, 256, bias=False)).to(DEV)
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
    try:
        built = build_native_muon_optimizers(model, lr=torch.tensor(0.02, device=DEV))
        import pan2_amd.optim.patch_muon as pm

        assert torch_muon._single_tensor_muon is pm._single_tensor_muon
        assert pm.NS_FORM == "gram", "the drop-in installs the reference's gram-form NS by default"
        x = torch.randn(8, 256, device=DEV)
        model(x).square().sum().backward()
        w0 = model[0].weight.detach().clone()
        for o in built["optimizers"].values():
            o.step()
        torch.cuda.synchronize()
        assert not torch.equal(model[0].weight.detach(), w0)
        assert torch.isfinite(model[0].weight).all()
    finally:
        torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = saved


def test_fused_step_without_nesterov_through_the_abi():
    """pm_muon_step with nesterov = 0 (the header's u = buf; PAN 2's patch
    asserts nesterov, so only the C ABI reaches it): the fused prologue's
    momentum is bit-exact against the oracle, and the update is NS(buf)
    within the fp64 gate, on engine, small and tall matrices."""
    shapes = [(512, 1024), (700, 300), (96, 2000)]
    lr = 0.02
    g = torch.Generator("cpu").manual_seed(77)
    init = [((torch.randn(*s, generator=g) * 0.02).numpy(), (torch.randn(*s, generator=g) * 1e-3).numpy(),
             (torch.randn(*s, generator=g) * 1e-3).numpy()) for s in shapes]
    ps = [torch.from_numpy(p).to(DEV) for p, _, _ in init]
    gs = [torch.from_numpy(gr).to(DEV) for _, gr, _ in init]
    bs = [torch.from_numpy(b).to(DEV) for _, _, b in init]
    ratios = [muon_ref.adjust_lr_ratio(None, s) for s in shapes]
    print(f"non-nesterov fused step {shapes}", flush=True)
    _lib.muon_step(ps, gs, bs, ratios, lr=lr, weight_decay=0.01, momentum=0.95, nesterov=False,
                   ns_coefficients=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7)
    torch.cuda.synchronize()
    for p, b, (p0, g0, b0), s, r in zip(ps, bs, init, shapes, ratios):
        _, ref_b, ref_o = muon_ref.muon_step(p0, g0, b0, lr=lr, weight_decay=0.01, nesterov=False,
                                             ns_precision="fp64")
        assert np.array_equal(b.cpu().numpy(), ref_b), s
        o_got = (p0.astype(np.float64) * (1 - lr * 0.01) - p.cpu().numpy()) / (lr * r)
        err = float(np.linalg.norm(o_got - ref_o) / np.linalg.norm(ref_o))
        assert err <= 2e-2, (s, err)
        # and it is NS of the momentum buffer, not of the Nesterov blend
        ref_o_nest = muon_ref.muon_step(p0, g0, b0, lr=lr, weight_decay=0.01, ns_precision="fp64")[2]
        assert np.linalg.norm(o_got - ref_o_nest) > np.linalg.norm(o_got - ref_o), s
