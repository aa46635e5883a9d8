"""The K-split of mid-size matrices (pan2_amd/csrc/pm_tiles.hpp::k_split), on
the GPU through the C ABI.

A matrix whose own tiles would leave most of the chip idle and whose
contraction is long (512 <= Mp, chunks of at least 1024 k; e.g. BASELINE
config 1's lone 1024 x 4096, whose gram contracts over 4096) runs each split
stage as chunk partials in fp32 and a reduce launch that adds them in chunk
order before the stage's epilogue. The split depends on the matrix's padded
shape only, so a matrix must step to the same bits alone, in any group and
across workspace groups; large matrices (Mp >= 4096) never split. Accuracy
against the fp64 oracle is also covered by the shape sweeps of
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
SPLIT_1 = (1024, 4096)     # its gram (K = 4096) splits 4 ways
SPLIT_2 = (600, 2000)      # Mp 768, Np 2048: its gram (K = 2048) splits 2 ways
UNSPLIT = (4096, 4096)


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
