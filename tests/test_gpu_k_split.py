"""The K-split of mid-size matrices (pan2_amd/csrc/pm_tiles.hpp::k_split), on
the GPU through the C ABI.

A matrix whose own tiles would leave most of the chip idle and whose
contraction is long (512 <= Mp, chunks of at least 1024 k; e.g. BASELINE
config 1's lone 1024 x 4096, whose gram contracts over 4096) runs each split
stage as chunk partials in fp32 and a reduce launch that adds them in chunk
order before the stage's epilogue. The split depends on the matrix's padded
shape only, so a matrix must step to the same bits alone, in any group and
across workspace groups; large matrices (Mp >= 4096) never split. Shapes with
Mp of 2048 and 3072 split their symmetric products and UPDATE / FINAL too;
a split FINAL's param step (run by the reduce launch) is checked bit for bit
against pm_newton_schulz's output on the same update. Accuracy against the
fp64 oracle is also covered by the shape sweeps of
test_gpu_kernels (1024 x 4096 and its transpose) and test_gpu_random_shapes
(short sides of 512 to 700 with long sides of 2048 or more split their grams).
"""
import numpy as np
import pytest
import torch

from oracle import muon_ref
from pan2_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
COEFFS = (3.4445, -4.7750, 2.0315)
SPLIT_1 = (1024, 4096)     # its gram (K = 4096) splits 4 ways
SPLIT_2 = (600, 2000)      # Mp 768, Np 2048: its gram (K = 2048) splits 2 ways
UNSPLIT = (4096, 4096)
# Shapes whose symmetric products (K = Mp) and UPDATE / FINAL (K = Mp) split
# too; chunks per tile of (GRAM, the symmetric products, UPDATE / FINAL):
ALL_STAGES = {
    (2048, 2048): (2, 2, 2),
    (2048, 4096): (4, 2, 2),
    (4096, 2048): (4, 2, 2),   # tall: transposed, the 2048 side contracted
    (3072, 3072): (2, 2, 1),   # 144 UPDATE tiles: two chunks would exceed one wave of 256 CUs
}


def k_split(mp, tiles, kt):
    """The split rule of pm_tiles.hpp::k_split, restated to name each shape's
    expected chunks (tests/native/tile_order_check.cpp pins the C++ rule)."""
    if mp < 512 or tiles <= 0 or kt % 4:
        return 1
    s = 1
    while 2 * s <= 4 and (kt // 4) % (2 * s) == 0 and kt // (2 * s) >= 16 and tiles * 2 * s <= 256:
        s *= 2
    return s


def stage_splits(shape):
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    mp, np_ = up(min(shape)), up(max(shape))
    nt = mp // 256
    tri = nt * (nt + 1) // 2
    return k_split(mp, tri, np_ // 64), k_split(mp, tri, mp // 64), k_split(mp, nt * (np_ // 256), mp // 64)


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g)


def run(xs, form, limit=0):
    outs = [torch.empty(x.shape, dtype=torch.bfloat16, device=DEV) for x in xs]
    _lib.newton_schulz_into(list(zip(xs, outs)), ns_form=form, workspace_limit=limit)
    return outs


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_split_matrices_step_to_the_same_bits_in_any_group(form):
    shapes = [SPLIT_1, UNSPLIT, SPLIT_2, (SPLIT_1[1], SPLIT_1[0])]
    xs = [seeded(s, 40 + i).to(DEV) for i, s in enumerate(shapes)]
    alone = [run([x], form)[0] for x in xs]
    together = run(xs, form)
    apart = run(xs, form, limit=1)  # each matrix in a workspace group of its own
    for i, s in enumerate(shapes):
        assert torch.equal(together[i], alone[i]), (s, "grouped")
        assert torch.equal(apart[i], alone[i]), (s, "workspace groups")
    again = run(xs, form)
    for i in range(len(shapes)):
        assert torch.equal(again[i], together[i]), "deterministic"


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_split_stages_run_reduce_launches(form):
    _lib.timing_enable(True)
    try:
        _lib.timing_read()
        run([seeded(SPLIT_1, 1).to(DEV)], form)
        split = _lib.timing_read()
        run([seeded(UNSPLIT, 2).to(DEV)], form)
        unsplit = _lib.timing_read()
    finally:
        _lib.timing_enable(False)
    n_gram = sum(1 for r in split if r["kind"] == "gram")
    n_reduce = sum(1 for r in split if r["kind"] == "reduce")
    print(f"{form}: 1024x4096 {n_gram} gram launches, {n_reduce} reduces", flush=True)
    assert n_reduce == n_gram > 0  # its grams split, its K = 1024 products do not
    # each reduce follows its gram
    kinds = [r["kind"] for r in split]
    assert all(kinds[i - 1] == "gram" for i, k in enumerate(kinds) if k == "reduce")
    assert not any(r["kind"] == "reduce" for r in unsplit)
    # the stage's FLOPs are counted once, on its GEMM launch
    assert all(r["flops"] == 0 for r in split if r["kind"] == "reduce")


def test_split_matrix_within_the_gate():
    """The lone config-1 matrix, its grams split, against the fp64 oracle
    (the north star's 2e-2)."""
    g = seeded(SPLIT_1, 7)
    out = run([g.to(DEV)], "standard")[0]
    ref = muon_ref.ns_standard(g.numpy(), precision="fp64")
    err = float(np.linalg.norm(out.float().cpu().numpy() - ref) / np.linalg.norm(ref))
    print(f"1024x4096 split grams: rel-Frobenius {err:.4f}", flush=True)
    assert err <= 2e-2


def test_split_table_matches_the_rule():
    assert {s: stage_splits(s) for s in ALL_STAGES} == ALL_STAGES
    assert stage_splits(SPLIT_1) == (4, 1, 1) and stage_splits(UNSPLIT) == (1, 1, 1)


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_every_split_stage_steps_to_the_same_bits_in_any_group(form):
    """Symmetric products and UPDATE / FINAL split as well as grams: each
    matrix alone, all in one group, each in a workspace group of its own."""
    shapes = list(ALL_STAGES) + [UNSPLIT, (300, 2000)]
    xs = [seeded(s, 60 + i).to(DEV) for i, s in enumerate(shapes)]
    alone = [run([x], form)[0] for x in xs]
    together = run(xs, form)
    apart = run(xs, form, limit=1)
    for i, s in enumerate(shapes):
        assert torch.equal(together[i], alone[i]), (s, "grouped")
        assert torch.equal(apart[i], alone[i]), (s, "workspace groups")


def test_every_split_stage_runs_its_reduce():
    """Standard form, one matrix a call: a reduce follows every stage launch
    whose matrix splits, and no other."""
    _lib.timing_enable(True)
    try:
        for shape, (sg, ss, sf) in ALL_STAGES.items():
            _lib.timing_read()
            run([seeded(shape, 5).to(DEV)], "standard")
            recs = _lib.timing_read()
            kinds = [r["kind"] for r in recs if r["kind"] not in ("prologue", "norm")]
            split = {"gram": sg > 1, "poly": ss > 1, "update": sf > 1, "final": sf > 1}
            want = []
            for k in [k for k in kinds if k != "reduce"]:
                want += [k, "reduce"] if split[k] else [k]
            print(f"{shape}: {kinds.count('reduce')} reduces in {len(kinds)} GEMM-side launches", flush=True)
            assert kinds == want, (shape, kinds)
    finally:
        _lib.timing_enable(False)


@pytest.mark.parametrize("shape", list(ALL_STAGES))
def test_split_stages_within_the_gate(shape):
    g = seeded(shape, 8)
    out = run([g.to(DEV)], "standard")[0]
    ref = muon_ref.ns_standard(g.numpy(), precision="fp64")
    err = float(np.linalg.norm(out.float().cpu().numpy() - ref) / np.linalg.norm(ref))
    print(f"{shape} split stages: rel-Frobenius {err:.4f}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("form", ["standard", "gram"])
@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_split_final_steps_params_as_its_ns_output_does(form, pdt):
    """pm_muon_step through a split FINAL (its param step in the reduce
    launch's epilogue) against pm_newton_schulz on the same momentum-blended
    update u and the param step of pan/optim/muon_triton.py:127-131, bit for
    bit: the prologue writes X = bf16(u) and its partials from the same values
    in both modes, so O is the same bf16 matrix."""
    lr, wd, mu = 0.02, 0.01, 0.95
    shapes = [(2048, 2048), (4096, 2048), (2048, 4096)]
    params, grads, bufs, ratios, init = [], [], [], [], []
    for i, s in enumerate(shapes):
        p0 = (seeded(s, 70 + 3 * i) * 0.02).to(pdt)
        g = seeded(s, 71 + 3 * i) * 1e-3
        b = seeded(s, 72 + 3 * i) * 1e-3
        params.append(p0.to(DEV))
        grads.append(g.to(DEV))
        bufs.append(b.to(DEV))
        ratios.append(muon_ref.adjust_lr_ratio(None, s))
        init.append((p0.float().numpy(), g.numpy(), b.numpy()))
    _lib.muon_step(params, grads, bufs, ratios, lr=lr, weight_decay=wd, momentum=mu, nesterov=True,
                   ns_coefficients=COEFFS, ns_steps=5, eps=1e-7, ns_form=form)
    us = [muon_ref.momentum_nesterov(b, g, mu, True) for _, g, b in init]
    outs = run([torch.from_numpy(u).to(DEV) for _, u in us], form)
    torch.cuda.synchronize()
    for i, s in enumerate(shapes):
        assert np.array_equal(bufs[i].cpu().numpy(), us[i][0]), (s, "momentum")
        ref = muon_ref.step_param(init[i][0], outs[i].float().cpu().numpy(), lr, wd, ratios[i])
        ref = torch.from_numpy(ref).to(pdt)
        assert torch.equal(params[i].cpu(), ref), (s, form, pdt)
