"""The workspace entry points captured in a HIP graph (torch.cuda.graph):
pm_muon_step, pm_newton_schulz and pm_adam_step put their descriptor tables
in as kernel arguments on a capturing stream, never as a copy from a pinned
staging buffer that later calls reuse. Every replay is checked bit for bit
against the same call made eagerly on a twin state, with eager library calls
(which do go through the staging buffers), a device lr change and a
synchronisation between replays. One eager call precedes each capture, so
the kernels' code object is loaded outside it.
"""

import pytest
import torch

from pan2_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
COEFFS = (3.4445, -4.7750, 2.0315)
# engine matrices (the 1024 x 4096's grams K-split: the reduce launch is
# captured too), small ones (short side <= 128), a tall one
SHAPES = [(1024, 4096), (300, 1000), (96, 2000), (2000, 64), (512, 512), (700, 300)]


def make_state(shapes, seed, pdt=torch.float32):
    g = torch.Generator("cpu").manual_seed(seed)
    ps, gs, bs = [], [], []
    for s in shapes:
        ps.append((torch.randn(*s, generator=g) * 0.02).to(DEV, pdt))
        gs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV, torch.bfloat16))
        bs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV))
    return ps, gs, bs


def step(state, lr, ns_form):
    ps, gs, bs = state
    ratios = [max(1.0, s.shape[0] / s.shape[1]) ** 0.5 for s in ps]
    _lib.muon_step(ps, gs, bs, ratios, lr=lr, weight_decay=0.01, momentum=0.95, nesterov=True,
                   ns_coefficients=COEFFS, ns_steps=5, eps=1e-7, ns_form=ns_form)


@pytest.mark.parametrize("ns_form", ["standard", "gram"])
def test_muon_step_captured_replays_the_eager_step(ns_form):
    lr = torch.tensor(0.02, device=DEV)
    step(make_state(SHAPES, 801), lr, ns_form)  # outside capture: kernels loaded
    torch.cuda.synchronize()
    ref, got = make_state(SHAPES, 800), make_state(SHAPES, 800)
    other = make_state([(256, 640), (128, 384)], 802)
    graph = torch.cuda.CUDAGraph()
    print(f"pm_muon_step graph capture {ns_form}: {SHAPES}", flush=True)
    with torch.cuda.graph(graph):
        assert torch.cuda.is_current_stream_capturing()  # what the library asks of the stream it is given
        step(got, lr, ns_form)
    torch.cuda.synchronize()
    for rep, lr_val in enumerate((0.02, 0.01, 0.03)):
        step(other, lr, ns_form)  # an eager call of other shapes reuses the staging buffers
        lr.fill_(lr_val)
        graph.replay()
        step(ref, lr, ns_form)
        torch.cuda.synchronize()
        for i in range(len(SHAPES)):
            assert torch.equal(got[0][i], ref[0][i]), f"param {i} after replay {rep}"
            assert torch.equal(got[2][i], ref[2][i]), f"momentum {i} after replay {rep}"
    graph.reset()


def test_newton_schulz_captured_matches_eager():
    g = torch.Generator("cpu").manual_seed(810)
    xs = [torch.randn(*s, generator=g).to(DEV, torch.bfloat16) for s in SHAPES]
    want = [torch.empty_like(x) for x in xs]
    got = [torch.empty_like(x) for x in xs]
    _lib.newton_schulz_into(list(zip(xs, want)), ns_coefficients=COEFFS)  # outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print(f"pm_newton_schulz graph capture: {SHAPES}", flush=True)
    with torch.cuda.graph(graph):
        assert torch.cuda.is_current_stream_capturing()
        _lib.newton_schulz_into(list(zip(xs, got)), ns_coefficients=COEFFS)
    for rep in range(2):
        for o in got:
            o.zero_()
        _lib.newton_schulz_into([(xs[0][:256], torch.empty_like(xs[0][:256]))], ns_coefficients=COEFFS)
        graph.replay()
        torch.cuda.synchronize()
        for i in range(len(xs)):
            assert torch.equal(got[i], want[i]), f"matrix {i} after replay {rep}"
    graph.reset()


def test_adam_step_captured_replays_the_eager_step():
    sizes = [8193, 100003, 5, 4096]
    kw = dict(beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.01, amsgrad=False, maximize=False, decoupled=True)

    def state(seed):
        g = torch.Generator("cpu").manual_seed(seed)
        ps = [(torch.randn(n, generator=g) * 0.5).to(DEV) for n in sizes]
        gs = [(torch.randn(n, generator=g) * 1e-2).to(DEV) for n in sizes]
        return (ps, gs, [torch.zeros_like(p) for p in ps], [torch.zeros_like(p) for p in ps],
                [torch.zeros((), device=DEV) for _ in ps])

    def adam(st, lr):
        ps, gs, ms, vs, steps = st
        _lib.adam_step(ps, gs, ms, vs, [], steps, lr=lr, **kw)

    lr = torch.tensor(1e-3, device=DEV)
    adam(state(820), lr)  # outside capture
    torch.cuda.synchronize()
    ref, got = state(821), state(821)
    graph = torch.cuda.CUDAGraph()
    print(f"pm_adam_step graph capture: {sizes}", flush=True)
    with torch.cuda.graph(graph):
        assert torch.cuda.is_current_stream_capturing()
        adam(got, lr)
    torch.cuda.synchronize()
    for rep, lr_val in enumerate((1e-3, 5e-4, 2e-3)):
        adam(state(822), lr)  # eager, through the staging buffers
        lr.fill_(lr_val)
        graph.replay()
        adam(ref, lr)
        torch.cuda.synchronize()
        for k in (0, 2, 3, 4):
            for i in range(len(sizes)):
                assert torch.equal(got[k][i], ref[k][i]), f"list {k} tensor {i} after replay {rep}"
    graph.reset()


def test_standalone_ops_captured_match_eager():
    """pm_gram and pm_gemm_symmetric (descriptor tables as kernel arguments
    under capture), pm_momentum_nesterov and pm_step_param (no table)."""
    g = torch.Generator("cpu").manual_seed(830)
    x = torch.randn(512, 768, generator=g).to(DEV, torch.bfloat16)
    a, b, d = (torch.randn(512, 512, generator=g).to(DEV, torch.bfloat16) for _ in range(3))
    buf0 = (torch.randn(300, 700, generator=g) * 1e-3).to(DEV)
    grad = (torch.randn(300, 700, generator=g) * 1e-3).to(DEV, torch.bfloat16)
    p0 = (torch.randn(300, 700, generator=g) * 0.02).to(DEV)
    lr = torch.tensor(0.02, device=DEV)

    def ops(buf, p):
        r = _lib.gram(x)
        s = _lib.gemm_symmetric(a, b, d, alpha=2.0, beta=-0.5)
        u = torch.empty_like(grad)
        _lib.momentum_nesterov_into(buf, grad, u, 0.95)
        _lib.step_param_inplace(p, u, lr, 0.01, 1.5)
        return r, s, u

    want = ops(buf0.clone(), p0.clone())  # outside capture
    torch.cuda.synchronize()
    buf, p = buf0.clone(), p0.clone()
    graph = torch.cuda.CUDAGraph()
    print("standalone ops graph capture", flush=True)
    with torch.cuda.graph(graph):
        assert torch.cuda.is_current_stream_capturing()
        got = ops(buf, p)
    _lib.gram(x[:256, :256].contiguous())  # an eager call through the staging buffers
    graph.replay()
    torch.cuda.synchronize()
    for i, (u, v) in enumerate(zip(got, want)):
        assert torch.equal(u, v), f"output {i}"
    ref_buf, ref_p = buf0.clone(), p0.clone()
    ops(ref_buf, ref_p)
    torch.cuda.synchronize()
    assert torch.equal(buf, ref_buf) and torch.equal(p, ref_p)
    graph.reset()
