"""GPU parity of the Adam / AdamW half of the step (pm_adam_step, behind
torch's fused Adam: pan/optim/muon.py:155-164, TORCH/optim/adam.py:803-898),
through the C ABI.

Tolerances:
- against the CPU oracle (oracle/adamw_ref.py, the same fp32 operations in the
  same order): exp_avg and exp_avg_sq bit-exact; the param within one ulp of
  its storage dtype (the bias corrections are double-precision pow on each
  side, whose last bit may differ);
- against torch's own fused Adam on the GPU: the oracle's bound against torch
  on the CPU (a few fp32 ulps of each array's scale), as the two use
  different operation orders.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import adamw_ref
from oracle.bf16 import round_bf16
from pan2_amd import _lib

pytestmark = pytest.mark.gpu

ADAM_MODULE = importlib.import_module("torch.optim.adam")

DEV = "cuda:0"
SIZES = [1, 7, 8, 9, 8191, 8192, 8193, 100003, 0, 64]
DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


def as_dtype(x, dt):
    if dt == "f16":
        return x.astype(np.float16).astype(np.float32)
    return round_bf16(x) if dt == "bf16" else x


def dev(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, DT[dt])


def ulp(x, dt):
    """Spacing of the storage dtype at x."""
    x = np.abs(np.asarray(x, dtype=np.float32))
    bits = {"bf16": 7, "f16": 10}.get(dt, 23)
    tiny = np.float32(2.0 ** -14) if dt == "f16" else np.float32(1e-38)  # fp16 subnormals are evenly spaced
    e = np.floor(np.log2(np.maximum(x, tiny)))
    return np.ldexp(1.0, (e - bits).astype(int))


def run_gpu(p0s, grads, *, dtypes=("f32", "f32", "f32", "f32"), lr=2e-3, lr_dev=False, betas=(0.95, 0.95),
            eps=1e-8, wd=0.05, decoupled=True, amsgrad=False, maximize=False):
    """Steps of pm_adam_step over the tensors; grads[k][i] is step k's grad of tensor i."""
    pdt, gdt, mdt, vdt = dtypes
    ps = [dev(as_dtype(p, pdt), pdt) for p in p0s]
    ms = [torch.zeros_like(p, dtype=DT[mdt]) for p in ps]
    vs = [torch.zeros_like(p, dtype=DT[vdt]) for p in ps]
    xs = [torch.zeros_like(p, dtype=DT[vdt]) for p in ps] if amsgrad else [None] * len(ps)
    steps = [torch.zeros((), dtype=torch.float32, device=DEV) for _ in ps]
    lr_arg = torch.tensor(lr, dtype=torch.float32, device=DEV) if lr_dev else lr
    for gk in grads:
        gs = [dev(as_dtype(g, gdt), gdt) for g in gk]
        _lib.adam_step(ps, gs, ms, vs, xs, steps, lr=lr_arg, beta1=betas[0], beta2=betas[1], eps=eps,
                       weight_decay=wd, amsgrad=amsgrad, maximize=maximize, decoupled=decoupled)
    torch.cuda.synchronize()
    host = lambda ts: [None if t is None else t.float().cpu().numpy() for t in ts]  # noqa: E731
    return host(ps), host(ms), host(vs), host(xs), [float(s) for s in steps]


def run_oracle(p0s, grads, *, dtypes=("f32", "f32", "f32", "f32"), lr=2e-3, betas=(0.95, 0.95), eps=1e-8, wd=0.05,
               decoupled=True, amsgrad=False, maximize=False):
    pdt, gdt, mdt, vdt = dtypes
    out = []
    for i, p0 in enumerate(p0s):
        p = as_dtype(p0, pdt)
        m, v = np.zeros_like(p), np.zeros_like(p)
        x = np.zeros_like(p) if amsgrad else None
        step = 0.0
        for gk in grads:
            p, m, v, x, step = adamw_ref.adam_step(p, as_dtype(gk[i], gdt), m, v, step, lr=lr, beta1=betas[0],
                                                   beta2=betas[1], eps=eps, weight_decay=wd, decoupled=decoupled,
                                                   amsgrad=amsgrad, max_exp_avg_sq=x, maximize=maximize,
                                                   dtypes=(pdt, mdt, vdt))
        out.append((p, m, v, x, step))
    return out


def case(seed=0, sizes=SIZES, steps=3):
    p0s = [rnd(n, seed + i, 0.5) for i, n in enumerate(sizes)]
    grads = [[rnd(n, 1000 * (k + 1) + seed + i, 10.0 ** (k - 2)) for i, n in enumerate(sizes)] for k in range(steps)]
    return p0s, grads


def assert_matches_oracle(got, want, pdt):
    ps, ms, vs, xs, steps = got
    for i, (p, m, v, x, step) in enumerate(want):
        assert steps[i] == step
        assert np.array_equal(ms[i], m), f"exp_avg of tensor {i}"
        assert np.array_equal(vs[i], v), f"exp_avg_sq of tensor {i}"
        if x is not None:
            assert np.array_equal(xs[i], x), f"max_exp_avg_sq of tensor {i}"
        assert np.all(np.abs(ps[i] - p) <= ulp(p, pdt)), f"param of tensor {i}: {np.abs(ps[i] - p).max()}"


def test_adamw_fp32_matches_oracle_on_ragged_sizes():
    print("adamw fp32 ragged", flush=True)
    p0s, grads = case(1)
    assert_matches_oracle(run_gpu(p0s, grads), run_oracle(p0s, grads), "f32")


@pytest.mark.parametrize("dtypes", [("bf16", "bf16", "f32", "f32"), ("bf16", "bf16", "bf16", "bf16"),
                                    ("f32", "bf16", "f32", "f32"), ("f16", "f16", "f16", "f16"),
                                    ("f16", "f16", "f32", "f32")])
def test_adamw_mixed_dtypes_match_oracle(dtypes):
    print(f"adamw dtypes {dtypes}", flush=True)
    p0s, grads = case(2, sizes=[9, 8193, 4096, 1])
    assert_matches_oracle(run_gpu(p0s, grads, dtypes=dtypes), run_oracle(p0s, grads, dtypes=dtypes), dtypes[0])


@pytest.mark.parametrize("variant", ["adam_l2", "amsgrad", "maximize", "no_decay", "wide_lerp"])
def test_adam_variants_match_oracle(variant):
    print(f"adam variant {variant}", flush=True)
    kw = {"adam_l2": dict(decoupled=False, wd=0.01, betas=(0.9, 0.999)),
          "amsgrad": dict(amsgrad=True, wd=0.1, betas=(0.8, 0.99)),
          "maximize": dict(maximize=True),
          "no_decay": dict(wd=0.0, betas=(0.9, 0.999)),
          "wide_lerp": dict(betas=(0.3, 0.6))}[variant]
    p0s, grads = case(3, sizes=[8193, 77, 16384], steps=4)
    assert_matches_oracle(run_gpu(p0s, grads, **kw), run_oracle(p0s, grads, **kw), "f32")


def test_device_lr_matches_host_lr():
    """The tensor-lr path reads lr on the device as fp32 (2e-3 is not exact
    there) and forms the decay factor 1 - lr*wd in fp32: the moments are
    identical, the param agrees to a few ulps of itself plus 1e-6 of lr."""
    p0s, grads = case(4, sizes=[8193, 100])
    lr = 2e-3
    a = run_gpu(p0s, grads, lr=lr)
    b = run_gpu(p0s, grads, lr=lr, lr_dev=True)
    for i in range(len(p0s)):
        assert np.array_equal(a[1][i], b[1][i]) and np.array_equal(a[2][i], b[2][i])
        assert np.all(np.abs(a[0][i] - b[0][i]) <= 4 * ulp(a[0][i], "f32") + 1e-6 * lr)


def _torch_vs_ours(torch_fused_adam, *, lr, grad_scale=None, found_inf=None, pdt=torch.float32, amsgrad=False,
                   decoupled=True, wd=0.05, steps=3, gscale=1e-2):
    """The same steps through torch's fused Adam and through the patched one, on copies."""
    from pan2_amd.optim import patch_adamw

    sizes = [8193, 100003, 5, 4096]
    pdts = list(pdt) if isinstance(pdt, (list, tuple)) else [pdt] * len(sizes)
    results = []
    for ours in (False, True):
        ps = [torch.from_numpy(rnd(n, 50 + i, 0.5)).to(DEV, pdts[i]) for i, n in enumerate(sizes)]
        ms = [torch.zeros_like(p) for p in ps]
        vs = [torch.zeros_like(p) for p in ps]
        xs = [torch.zeros_like(p) for p in ps] if amsgrad else []
        st = [torch.zeros((), dtype=torch.float32, device=DEV) for _ in ps]
        gs_all = []
        for k in range(steps):
            gs = [torch.from_numpy(rnd(n, 70 + 10 * k + i, gscale)).to(DEV, pdts[i]) for i, n in enumerate(sizes)]
            kw = dict(amsgrad=amsgrad, has_complex=False, beta1=0.95, beta2=0.95, lr=lr, weight_decay=wd, eps=1e-8,
                      maximize=False, capturable=False, differentiable=False, decoupled_weight_decay=decoupled)
            if ours:
                patch_adamw._fused_adam(ps, gs, ms, vs, xs, st, grad_scale, found_inf, **kw)
            else:
                with torch_fused_adam():
                    ADAM_MODULE._fused_adam(ps, gs, ms, vs, xs, st, grad_scale, found_inf, **kw)
            gs_all.append(gs)
        torch.cuda.synchronize()
        f = lambda ts: [t.float().cpu().numpy() for t in ts]  # noqa: E731
        results.append((f(ps), f(ms), f(vs), f(xs), [float(s) for s in st], [f(g) for g in gs_all]))
    return results


def _close(a, b, what):
    assert np.all(np.abs(a - b) <= 2e-6 * np.abs(b) + 1e-6 * np.abs(b).max()), what


@pytest.mark.parametrize("lr_kind", ["float", "device"])
def test_matches_torch_fused_adamw(torch_fused_adam, lr_kind):
    print(f"vs torch fused adamw lr={lr_kind}", flush=True)
    lr = 2e-3 if lr_kind == "float" else torch.tensor(2e-3, device=DEV)
    (tp, tm, tv, _, tst, _), (p, m, v, _, st, _) = _torch_vs_ours(torch_fused_adam, lr=lr)
    assert st == tst
    for i in range(len(p)):
        _close(m[i], tm[i], f"exp_avg {i}")
        _close(v[i], tv[i], f"exp_avg_sq {i}")
        assert np.all(np.abs(p[i] - tp[i]) <= 2e-6 * np.abs(tp[i]) + 2e-6 * 2e-3), f"param {i}"


def test_matches_torch_fused_adam_amsgrad_and_bf16(torch_fused_adam):
    (tp, tm, tv, tx, tst, _), (p, m, v, x, st, _) = _torch_vs_ours(torch_fused_adam, lr=1e-3, amsgrad=True,
                                                                   pdt=torch.bfloat16, decoupled=False, wd=0.01)
    assert st == tst
    for i in range(len(p)):
        # bf16 storage: one bf16 rounding of values that agree to a few fp32 ulps
        for a, b in ((m[i], tm[i]), (v[i], tv[i]), (x[i], tx[i]), (p[i], tp[i])):
            assert np.all(np.abs(a - b) <= ulp(b, "bf16") + 1e-6 * np.abs(b).max())


def test_mixed_dtype_lists_match_torch_fused_adam(torch_fused_adam):
    """One call whose lists mix fp32, bf16 and fp16 tensors (each with state of
    its param's dtype): torch's fused Adam splits them by dtype, the patched one
    takes them in one launch with a dtype code per tensor."""
    pdts = [torch.float32, torch.bfloat16, torch.float16, torch.float32]
    (tp, tm, tv, _, tst, _), (p, m, v, _, st, _) = _torch_vs_ours(torch_fused_adam, lr=1e-3, pdt=pdts, gscale=1.0)
    assert st == tst
    for i, dt in enumerate(("f32", "bf16", "f16", "f32")):
        for a, b in ((m[i], tm[i]), (v[i], tv[i]), (p[i], tp[i])):
            tol = 2e-6 * np.abs(b) if dt == "f32" else ulp(b, dt)
            assert np.all(np.abs(a - b) <= tol + 1e-6 * np.abs(b).max()), (i, dt)


def test_matches_torch_fused_adam_fp16(torch_fused_adam):
    """fp16 params and state, as torch's fused Adam takes them (TORCH/optim/adam.py:803-898).
    Grads of order 1 keep exp_avg_sq out of fp16's subnormal range, where the
    spacing is so coarse that one stored ulp of difference (the two kernels
    order their fp32 operations differently) moves sqrt(v) by tens of percent
    on the next step; bit-exactness against the oracle covers that range."""
    (tp, tm, tv, _, tst, _), (p, m, v, _, st, _) = _torch_vs_ours(torch_fused_adam, lr=1e-3, pdt=torch.float16,
                                                                  gscale=1.0)
    assert st == tst
    for i in range(len(p)):
        for a, b in ((m[i], tm[i]), (v[i], tv[i]), (p[i], tp[i])):
            assert np.all(np.abs(a - b) <= ulp(b, "f16") + 1e-6 * np.abs(b).max())


def test_unsupported_tensors_go_to_torchs_fused_adam(torch_fused_adam):
    """float64 device tensors and CPU tensors are left to torch's own fused Adam,
    bit for bit what an unpatched process computes; the fp32 device tensors of
    the same call still run on libpanmuon."""
    from pan2_amd.optim import patch_adamw

    def state(specs, seed):
        out = []
        for i, (dev_, dt, n) in enumerate(specs):
            g = torch.Generator().manual_seed(seed + i)
            p = (torch.randn(n, generator=g, dtype=torch.float64) * 0.5).to(dev_, dt)
            out.append((p, torch.zeros_like(p), torch.zeros_like(p), torch.zeros((), device=dev_)))
        return out

    specs = [(DEV, torch.float64, 1000), ("cpu", torch.float32, 777), (DEV, torch.float32, 4096)]
    kw = dict(amsgrad=False, has_complex=False, beta1=0.9, beta2=0.99, lr=1e-3, weight_decay=0.01, eps=1e-8,
              maximize=False, capturable=False, differentiable=False, decoupled_weight_decay=True)
    runs = []
    for ours in (False, True):
        st = state(specs, 5)
        for k in range(2):
            gs = [torch.full_like(p, 1e-2 * (k + 1)) for p, *_ in st]
            lists = [list(x) for x in zip(*st)]
            if ours:
                patch_adamw._fused_adam(lists[0], gs, lists[1], lists[2], [], lists[3], None, None, **kw)
            else:
                with torch_fused_adam():
                    ADAM_MODULE._fused_adam(lists[0], gs, lists[1], lists[2], [], lists[3], None, None, **kw)
        torch.cuda.synchronize()
        runs.append([[t.double().cpu() for t in s] for s in st])
    for i in range(2):  # torch's own kernel on both sides
        for a, b in zip(runs[0][i], runs[1][i]):
            assert torch.equal(a, b), i
    p_t, p_o = runs[0][2][0], runs[1][2][0]  # fp32 on the device: ours, against torch's within fp32 ulps
    assert torch.all((p_t - p_o).abs() <= 2e-6 * p_t.abs() + 1e-9)


def test_noncontiguous_tensors_go_to_torchs_fused_adam(torch_fused_adam):
    """A transposed param (its state and grad of the same strides, as torch's
    zeros_like and autograd make them) is not walked as a flat array by
    pm_adam_step: torch's own fused Adam steps it, bit for bit what an
    unpatched process computes; the contiguous param of the same call still
    runs on libpanmuon."""
    from pan2_amd.optim import patch_adamw

    kw = dict(amsgrad=True, has_complex=False, beta1=0.9, beta2=0.99, lr=1e-3, weight_decay=0.01, eps=1e-8,
              maximize=False, capturable=False, differentiable=False, decoupled_weight_decay=True)
    runs = []
    for ours in (False, True):
        gen = torch.Generator().manual_seed(17)
        ps = [torch.randn(48, 64, generator=gen).to(DEV).t(), torch.randn(4096, generator=gen).to(DEV)]
        assert not ps[0].is_contiguous()
        ms, vs, xs = ([torch.zeros_like(p) for p in ps] for _ in range(3))
        st = [torch.zeros((), device=DEV) for _ in ps]
        for k in range(2):
            gs = [(torch.randn(p.shape, generator=gen) * 1e-2).to(DEV) for p in ps]
            gs[0] = torch.empty_like(ps[0]).copy_(gs[0])  # the param's strides, as autograd gives
            if ours:
                patch_adamw._fused_adam(ps, gs, ms, vs, xs, st, None, None, **kw)
            else:
                with torch_fused_adam():
                    ADAM_MODULE._fused_adam(ps, gs, ms, vs, xs, st, None, None, **kw)
        torch.cuda.synchronize()
        runs.append([[t.cpu() for t in ts] for ts in (ps, ms, vs, xs)] + [[float(s) for s in st]])
    for a, b in zip(runs[0][:4], runs[1][:4]):  # the transposed param: torch's kernel on both sides
        assert torch.equal(a[0], b[0])
    assert runs[0][4] == runs[1][4] == [2.0, 2.0]
    p_t, p_o = runs[0][0][1], runs[1][0][1]
    assert torch.all((p_t - p_o).abs() <= 2e-6 * p_t.abs() + 1e-9)


def test_found_inf_skips_like_torch(torch_fused_adam):
    """A GradScaler's found_inf = 1 leaves params, moments and steps untouched; 0 steps normally."""
    for flag in (1.0, 0.0):
        fi = torch.tensor(flag, device=DEV)
        (tp, tm, tv, _, tst, _), (p, m, v, _, st, _) = _torch_vs_ours(torch_fused_adam, lr=2e-3, found_inf=fi,
                                                                      steps=2)
        assert st == tst == [2.0 * (1 - flag)] * 4
        for i in range(len(p)):
            if flag:
                assert np.array_equal(p[i], tp[i]) and not np.any(m[i]) and not np.any(v[i])
            else:
                _close(m[i], tm[i], "exp_avg")


def test_grad_scale_like_torch(torch_fused_adam):
    gs = torch.tensor(1024.0, device=DEV)
    (tp, tm, tv, _, tst, tg), (p, m, v, _, st, g) = _torch_vs_ours(torch_fused_adam, lr=2e-3, grad_scale=gs)
    for i in range(len(p)):
        _close(m[i], tm[i], "exp_avg")
        _close(v[i], tv[i], "exp_avg_sq")
    for k in range(len(g)):  # the grads are left as torch leaves them
        for i in range(len(g[k])):
            assert np.array_equal(g[k][i], tg[k][i]), (k, i)


def test_factory_adamw_runs_on_libpanmuon_and_round_trips_state():
    """With a tensor lr the factory installs the HIP AdamW; its state is
    torch's own, so a state_dict round trip continues bit-identically."""
    import copy

    from pan2_amd.optim import patch_adamw
    from pan2_amd.optim.muon import build_native_muon_optimizers

    def model():
        torch.manual_seed(0)
        m = torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.LayerNorm(512), torch.nn.Linear(512, 256))
        return m.to(DEV)

    def grads(mod, k):
        g = torch.Generator(device="cpu").manual_seed(100 + k)
        for p in mod.parameters():
            p.grad = (torch.randn(p.shape, generator=g) * 1e-2).to(DEV)

    a = model()
    adamw = build_native_muon_optimizers(a, lr=torch.tensor(1e-3, device=DEV), weight_decay=0.05)["optimizers"]["adamw"]
    assert ADAM_MODULE._fused_adam is patch_adamw._fused_adam
    for k in range(2):
        grads(a, k)
        adamw.step()
    torch.cuda.synchronize()
    state = copy.deepcopy(adamw.state_dict())
    snapshot = [p.detach().clone() for p in a.parameters()]
    for k in range(2, 4):
        grads(a, k)
        adamw.step()
    torch.cuda.synchronize()

    b = model()
    with torch.no_grad():
        for pb, ps in zip(b.parameters(), snapshot):
            pb.copy_(ps)
    adamw_b = build_native_muon_optimizers(b, lr=torch.tensor(1e-3, device=DEV), weight_decay=0.05)["optimizers"]["adamw"]
    adamw_b.load_state_dict(state)
    for k in range(2, 4):
        grads(b, k)
        adamw_b.step()
    torch.cuda.synchronize()
    moved = 0
    for pa, pb, ps in zip(a.parameters(), b.parameters(), snapshot):
        assert torch.equal(pa, pb)
        moved += int(not torch.equal(pa, ps))
    assert moved == 4  # the AdamW params (two biases, the LayerNorm weight and bias) moved; not the Muon weights
