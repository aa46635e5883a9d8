"""pm_muon_step_noalloc through the C ABI: the allocation-free variant of
pm_muon_step (a static device scratch instead of a caller workspace; the
descriptor tables as kernel arguments) gives bit-identical params and momentum
buffers to pm_muon_step on the same inputs. Two calls in a row, the second
with a smaller input that runs in the scratch the first call left behind.
"""

import pytest
import torch

from pan2_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
COEFFS = (3.4445, -4.7750, 2.0315)


def make_state(shapes, seed, pdt):
    """(params, grads, bufs) on the device; fp32 momentum, bf16 grads."""
    g = torch.Generator("cpu").manual_seed(seed)
    ps, gs, bs = [], [], []
    for s in shapes:
        ps.append((torch.randn(*s, generator=g) * 0.02).to(DEV, pdt))
        gs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV, torch.bfloat16))
        bs.append((torch.randn(*s, generator=g) * 1e-3).to(DEV))
    return ps, gs, bs


def step(state, *, noalloc, lr, ns_form):
    ps, gs, bs = state
    ratios = [max(1.0, s.shape[0] / s.shape[1]) ** 0.5 for s in ps]
    _lib.muon_step(ps, gs, bs, ratios, lr=lr, weight_decay=0.01, momentum=0.95, nesterov=True,
                   ns_coefficients=COEFFS, ns_steps=5, eps=1e-7, ns_form=ns_form, noalloc=noalloc)


@pytest.mark.parametrize("ns_form", ["standard", "gram"])
def test_noalloc_matches_workspace_step_twice(ns_form):
    # large, ragged and small (short side <= 128) matrices, fp32 and bf16 params,
    # so the first call runs several groups in the scratch; the call splits its
    # grams and the 2048 x 2048 symmetric products (partials in the scratch too)
    calls = [
        ([(1024, 4096), (700, 300), (96, 2000), (300, 1000), (2000, 64), (512, 512), (2048, 2048)], torch.float32),
        ([(256, 640), (100, 260)], torch.bfloat16),
    ]
    lr = torch.tensor(0.02, device=DEV)
    for k, (shapes, pdt) in enumerate(calls):
        print(f"noalloc {ns_form} call {k}: {shapes} {pdt}", flush=True)
        ref = make_state(shapes, 100 + k, pdt)
        got = make_state(shapes, 100 + k, pdt)
        step(ref, noalloc=False, lr=lr, ns_form=ns_form)
        step(got, noalloc=True, lr=lr, ns_form=ns_form)
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            assert torch.equal(got[0][i], ref[0][i]), f"param {i} of call {k}"
            assert torch.equal(got[2][i], ref[2][i]), f"momentum {i} of call {k}"
            assert not torch.equal(got[0][i], make_state(shapes, 100 + k, pdt)[0][i])  # the step moved it


@pytest.mark.parametrize("ns_form", ["standard", "gram"])
def test_noalloc_many_small_matrices_fused_gram(ns_form):
    """Enough small matrices for the fused gram (each apply forms the next R):
    the same bits from the scratch as from a workspace."""
    shapes = [(128, 256)] * 150 + [(200, 96)] * 150
    lr = torch.tensor(0.02, device=DEV)
    print(f"noalloc fused gram {ns_form}: {len(shapes)} small matrices", flush=True)
    ref = make_state(shapes, 300, torch.bfloat16)
    got = make_state(shapes, 300, torch.bfloat16)
    step(ref, noalloc=False, lr=lr, ns_form=ns_form)
    step(got, noalloc=True, lr=lr, ns_form=ns_form)
    torch.cuda.synchronize()
    for i in range(len(shapes)):
        assert torch.equal(got[0][i], ref[0][i]), f"param {i}"
        assert torch.equal(got[2][i], ref[2][i]), f"momentum {i}"


def test_noalloc_rejects_a_matrix_beyond_the_scratch_untouched():
    """A matrix whose workspace exceeds the scratch fails with PM_EWORKSPACE
    before anything is enqueued: the other matrix of the call is not stepped."""
    shapes = [(256, 512), (5120, 8192)]  # the second needs ~0.4 GB of workspace
    state = make_state(shapes, 7, torch.float32)
    before = [t.clone() for t in state[0]] + [t.clone() for t in state[2]]
    with pytest.raises(RuntimeError, match="PM_NOALLOC_SCRATCH_BYTES"):
        step(state, noalloc=True, lr=0.02, ns_form="standard")
    torch.cuda.synchronize()
    for a, b in zip(state[0] + state[2], before):
        assert torch.equal(a, b)


def test_noalloc_takes_a_matrix_that_fits_unsplit():
    """A lone 3584 x 6144 in the gram form fits the scratch unsplit (206 MiB);
    its K-split partials would not, so the call does not split it, and the
    scratch step equals the workspace step."""
    shapes = [(3584, 6144)]
    lr = torch.tensor(0.02, device=DEV)
    ref = make_state(shapes, 900, torch.bfloat16)
    got = make_state(shapes, 900, torch.bfloat16)
    step(ref, noalloc=False, lr=lr, ns_form="gram")
    step(got, noalloc=True, lr=lr, ns_form="gram")
    torch.cuda.synchronize()
    assert torch.equal(got[0][0], ref[0][0]) and torch.equal(got[2][0], ref[2][0])


def test_noalloc_allocates_nothing_through_torch():
    """The call takes no memory from torch's caching allocator (the scratch is
    the library's static array)."""
    shapes = [(512, 1536), (64, 700)]
    state = make_state(shapes, 11, torch.float32)
    step(state, noalloc=True, lr=0.02, ns_form="standard")  # the device's first call looks up the scratch
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(DEV)["allocation.all.allocated"]
    step(state, noalloc=True, lr=0.02, ns_form="standard")
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(DEV)["allocation.all.allocated"] == before


@pytest.mark.parametrize("ns_form", ["standard", "gram"])
def test_noalloc_step_captured_in_a_graph_replays_the_eager_step(ns_form):
    """pm_muon_step_noalloc captured with torch.cuda.graph after one eager call
    (the device's first call looks up the scratch, which must not happen under
    capture): every replay steps params and momentum to the same bits as an
    eager workspace step on a twin state. Eager work and a synchronisation sit
    between replays, and the device lr is changed between them (the graph reads
    it on the device)."""
    shapes = [(1024, 4096), (300, 1000), (96, 2000), (2000, 64), (512, 512)]
    lr = torch.tensor(0.02, device=DEV)
    warm = make_state(shapes, 501, torch.float32)
    step(warm, noalloc=True, lr=lr, ns_form=ns_form)
    torch.cuda.synchronize()
    ref = make_state(shapes, 500, torch.float32)
    got = make_state(shapes, 500, torch.float32)
    graph = torch.cuda.CUDAGraph()
    print(f"noalloc graph capture {ns_form}: {shapes}", flush=True)
    with torch.cuda.graph(graph):
        step(got, noalloc=True, lr=lr, ns_form=ns_form)
    torch.cuda.synchronize()
    for rep, lr_val in enumerate((0.02, 0.01, 0.03)):
        lr.fill_(lr_val)
        graph.replay()
        step(ref, noalloc=False, lr=lr, ns_form=ns_form)
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            assert torch.equal(got[0][i], ref[0][i]), f"param {i} after replay {rep}"
            assert torch.equal(got[2][i], ref[2][i]), f"momentum {i} after replay {rep}"
    graph.reset()
