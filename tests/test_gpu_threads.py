"""libpanmuon called from several host threads at once, each on its own
stream: ctypes releases the GIL around the foreign calls, so the library's
host code (descriptor tables, the pinned staging pool, launch planning) runs
concurrently. Every thread's results equal the same calls made one after
another on the default stream, bit for bit.
"""

import threading

import pytest
import torch

from pan2_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
COEFFS = (3.4445, -4.7750, 2.0315)
MUON_SHAPES = {
    "standard": [(1024, 4096), (300, 1000), (96, 2000), (512, 512)],
    "gram": [(512, 1536), (2000, 64), (700, 300), (128, 384)],
}
ADAM_SIZES = [8193, 100003, 5, 4096]


def muon_state(shapes, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    ps, gs, bs = [], [], []
    for s in shapes:
        ps.append((torch.randn(*s, generator=g) * 0.02).to(DEV))
        gs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV, torch.bfloat16))
        bs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV))
    return ps, gs, bs


def adam_state(seed):
    g = torch.Generator("cpu").manual_seed(seed)
    ps = [(torch.randn(n, generator=g) * 0.5).to(DEV) for n in ADAM_SIZES]
    gs = [(torch.randn(n, generator=g) * 1e-2).to(DEV) for n in ADAM_SIZES]
    return (ps, gs, [torch.zeros_like(p) for p in ps], [torch.zeros_like(p) for p in ps],
            [torch.zeros((), device=DEV) for _ in ps])


def muon_steps(state, form, n):
    ps, gs, bs = state
    ratios = [max(1.0, p.shape[0] / p.shape[1]) ** 0.5 for p in ps]
    for _ in range(n):
        _lib.muon_step(ps, gs, bs, ratios, lr=0.02, weight_decay=0.01, momentum=0.95, nesterov=True,
                       ns_coefficients=COEFFS, ns_steps=5, eps=1e-7, ns_form=form)


def adam_steps(state, n):
    ps, gs, ms, vs, steps = state
    for _ in range(n):
        _lib.adam_step(ps, gs, ms, vs, [], steps, lr=1e-3, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.01,
                       amsgrad=False, maximize=False, decoupled=True)


def test_concurrent_threads_on_own_streams_match_sequential_calls():
    n = 4
    jobs = {
        "standard": lambda st: muon_steps(st, "standard", n),
        "gram": lambda st: muon_steps(st, "gram", n),
        "adam": lambda st: adam_steps(st, n),
    }
    make = {
        "standard": lambda: muon_state(MUON_SHAPES["standard"], 900),
        "gram": lambda: muon_state(MUON_SHAPES["gram"], 901),
        "adam": lambda: adam_state(902),
    }
    ref = {k: make[k]() for k in jobs}
    for k, job in jobs.items():  # one after another, default stream
        job(ref[k])
    got = {k: make[k]() for k in jobs}
    torch.cuda.synchronize()
    streams = {k: torch.cuda.Stream(device=DEV) for k in jobs}
    start = threading.Barrier(len(jobs))
    errors = []

    def worker(k):
        try:
            start.wait()
            with torch.cuda.stream(streams[k]):
                jobs[k](got[k])
        except BaseException as e:  # surfaced below
            errors.append((k, e))

    print(f"threads: {sorted(jobs)}, {n} calls each", flush=True)
    threads = [threading.Thread(target=worker, args=(k,)) for k in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
    for k in jobs:
        for a_list, b_list in zip(got[k], ref[k]):
            for i, (a, b) in enumerate(zip(a_list, b_list)):
                assert torch.equal(a, b), f"{k}: tensor {i}"
