"""The K-split of mid-size matrices (pan2_amd/csrc/pm_tiles.hpp::k_split,
chosen per call by pan2_amd/csrc/panmuon.hip::split_call), on the GPU through
the C ABI.

A call whose engine matrices hold so few tiles of a stage that most of the
chip would sit idle (e.g. BASELINE config 1's lone 1024 x 4096, whose gram
has 10 tiles over K = 4096) runs that stage's tiles as chunks of the
contraction with fp32 partials, then a reduce launch that adds them in chunk
order before the stage's epilogue. A call that fills the chip does not split
(its partials would cost more than the idle CUs they fill). The choice
depends on the call only: one call gives the same bits in any workspace
grouping, and again on a second run. A matrix may round differently alone
and in a larger call, within the same gates. Shapes with Mp of 2048 and 3072
split their symmetric products and UPDATE / FINAL too when alone; a split
FINAL's param step (run by the reduce launch) is checked bit for bit against
pm_newton_schulz's output on the same update. Large matrices (Mp >= 4096)
never split.
"""
import numpy as np
import pytest
import torch

from oracle import muon_ref
from pan2_amd import _lib
from tests.ksplit_rule import call_splits

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
COEFFS = (3.4445, -4.7750, 2.0315)
SPLIT_1 = (1024, 4096)     # alone, its gram (K = 4096) splits 4 ways
SPLIT_2 = (600, 2000)      # Mp 768, Np 2048: alone, its gram (K = 2048) splits 2 ways
UNSPLIT = (4096, 4096)
# Alone, these split their symmetric products (K = Mp) and UPDATE / FINAL (K = Mp)
# too; chunks per tile of (GRAM, the symmetric products, UPDATE / FINAL):
ALL_STAGES = {
    (2048, 2048): (2, 2, 2),
    (2048, 4096): (4, 2, 2),
    (4096, 2048): (4, 2, 2),   # tall: transposed, the 2048 side contracted
    (3072, 3072): (2, 2, 1),   # 144 UPDATE tiles: two chunks would exceed one wave of 256 CUs
}


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g)


def run(xs, form, limit=0):
    outs = [torch.empty(x.shape, dtype=torch.bfloat16, device=DEV) for x in xs]
    _lib.newton_schulz_into(list(zip(xs, outs)), ns_form=form, workspace_limit=limit)
    return outs


def kinds_of(xs, form):
    _lib.timing_enable(True)
    try:
        _lib.timing_read()
        run(xs, form)
        return [r["kind"] for r in _lib.timing_read()]
    finally:
        _lib.timing_enable(False)


def rel_err(out, x):
    ref = muon_ref.ns_standard(x.cpu().numpy(), precision="fp64")
    return float(np.linalg.norm(out.float().cpu().numpy() - ref) / np.linalg.norm(ref))


def test_split_table_matches_the_rule():
    assert {s: call_splits([s])[0] for s in ALL_STAGES} == ALL_STAGES
    assert call_splits([SPLIT_1]) == [(4, 1, 1)] and call_splits([UNSPLIT]) == [(1, 1, 1)]
    assert call_splits([SPLIT_1, UNSPLIT]) == [(1, 1, 1)] * 2  # 146 gram tiles: the call fills the chip
    assert call_splits([(2048, 2048)] * 2) == [(2, 2, 2)] * 2 and call_splits([(2048, 2048)] * 48) == [(1, 1, 1)] * 48


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_a_call_gives_the_same_bits_in_any_workspace_grouping(form):
    """Split and unsplit matrices in one call, that call again with each matrix
    in a workspace group of its own, and once more: the same bits. Alone, each
    matrix splits as its shape allows: the same bits where that choice is the
    call's, within the north star's 2e-2 of the fp64 oracle either way."""
    for shapes in ([SPLIT_1, SPLIT_2, (SPLIT_1[1], SPLIT_1[0])],                 # the call splits (26 gram tiles)
                   [SPLIT_1, UNSPLIT, SPLIT_2, (SPLIT_1[1], SPLIT_1[0])],        # it does not (162)
                   list(ALL_STAGES)[:2] + [(300, 2000)]):
        xs = [seeded(s, 40 + i).to(DEV) for i, s in enumerate(shapes)]
        together = run(xs, form)
        apart = run(xs, form, limit=1)
        again = run(xs, form)
        call = call_splits(shapes)
        print(f"{form} {shapes}: chunks {call}", flush=True)
        for i, s in enumerate(shapes):
            assert torch.equal(apart[i], together[i]), (s, "workspace groups")
            assert torch.equal(again[i], together[i]), (s, "deterministic")
            alone = run([xs[i]], form)[0]
            if call_splits([s])[0] == call[i]:
                assert torch.equal(alone, together[i]), (s, "alone")
            elif form == "standard":
                assert rel_err(alone, xs[i]) <= 2e-2 and rel_err(together[i], xs[i]) <= 2e-2, s


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_split_stages_run_reduce_launches(form):
    split = kinds_of([seeded(SPLIT_1, 1).to(DEV)], form)
    unsplit = kinds_of([seeded(UNSPLIT, 2).to(DEV)], form)
    n_gram, n_reduce = split.count("gram"), split.count("reduce")
    print(f"{form}: 1024x4096 {n_gram} gram launches, {n_reduce} reduces", flush=True)
    assert n_reduce == n_gram > 0  # its grams split, its K = 1024 products do not
    assert all(split[i - 1] == "gram" for i, k in enumerate(split) if k == "reduce")  # each reduce follows its gram
    assert "reduce" not in unsplit


def test_a_call_that_fills_the_chip_does_not_split():
    """48 matrices of 2048 x 2048 (1728 gram tiles) run no reduce launch; one
    or two of them (36, 72 tiles) split every stage."""
    xs = [seeded((2048, 2048), 500 + i).to(DEV) for i in range(48)]
    many = kinds_of(xs, "standard")
    one = kinds_of(xs[:1], "standard")
    two = kinds_of(xs[:2], "standard")
    print(f"reduces: 48 matrices {many.count('reduce')}, one {one.count('reduce')}, two {two.count('reduce')}",
          flush=True)
    assert "reduce" not in many
    assert one.count("reduce") == two.count("reduce") == 15


def test_split_matrix_within_the_gate():
    """The lone config-1 matrix, its grams split, against the fp64 oracle
    (the north star's 2e-2)."""
    g = seeded(SPLIT_1, 7)
    err = rel_err(run([g.to(DEV)], "standard")[0], g)
    print(f"1024x4096 split grams: rel-Frobenius {err:.4f}", flush=True)
    assert err <= 2e-2


def test_every_split_stage_runs_its_reduce():
    """Standard form, one matrix a call: a reduce follows every stage launch
    whose matrix splits, and no other."""
    for shape, (sg, ss, sf) in ALL_STAGES.items():
        kinds = [k for k in kinds_of([seeded(shape, 5).to(DEV)], "standard") if k not in ("prologue", "norm")]
        split = {"gram": sg > 1, "poly": ss > 1, "update": sf > 1, "final": sf > 1}
        want = []
        for k in [k for k in kinds if k != "reduce"]:
            want += [k, "reduce"] if split[k] else [k]
        print(f"{shape}: {kinds.count('reduce')} reduces in {len(kinds)} GEMM-side launches", flush=True)
        assert kinds == want, (shape, kinds)


@pytest.mark.parametrize("shape", list(ALL_STAGES))
def test_split_stages_within_the_gate(shape):
    g = seeded(shape, 8)
    err = rel_err(run([g.to(DEV)], "standard")[0], g)
    print(f"{shape} split stages: rel-Frobenius {err:.4f}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("form", ["standard", "gram"])
@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_split_final_steps_params_as_its_ns_output_does(form, pdt):
    """pm_muon_step through a split FINAL (its param step in the reduce
    launch's epilogue; one matrix a call, so every stage splits) against
    pm_newton_schulz on the same momentum-blended update u and the param step
    of pan/optim/muon_triton.py:127-131, bit for bit: the prologue writes
    X = bf16(u) and its partials from the same values in both modes, so O is
    the same bf16 matrix."""
    lr, wd, mu = 0.02, 0.01, 0.95
    for i, s in enumerate([(2048, 2048), (4096, 2048), (2048, 4096)]):
        assert call_splits([s])[0][2] == 2
        p0 = (seeded(s, 70 + 3 * i) * 0.02).to(pdt)
        g = seeded(s, 71 + 3 * i) * 1e-3
        b = seeded(s, 72 + 3 * i) * 1e-3
        param, grad, buf = p0.to(DEV), g.to(DEV), b.to(DEV)
        ratio = muon_ref.adjust_lr_ratio(None, s)
        _lib.muon_step([param], [grad], [buf], [ratio], lr=lr, weight_decay=wd, momentum=mu, nesterov=True,
                       ns_coefficients=COEFFS, ns_steps=5, eps=1e-7, ns_form=form)
        new_buf, u = muon_ref.momentum_nesterov(b.numpy(), g.numpy(), mu, True)
        out = run([torch.from_numpy(u).to(DEV)], form)[0]
        torch.cuda.synchronize()
        assert np.array_equal(buf.cpu().numpy(), new_buf), (s, "momentum")
        ref = muon_ref.step_param(p0.float().numpy(), out.float().cpu().numpy(), lr, wd, ratio)
        assert torch.equal(param.cpu(), torch.from_numpy(ref).to(pdt)), (s, form, pdt)
