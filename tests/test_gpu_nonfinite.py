"""Non-finite inputs through the C ABI, both NS forms, engine and small-matrix
paths.

torch's _zeropower_via_newtonschulz (TORCH/optim/_muon.py:55-70) turns one
±Inf or NaN anywhere in its input into an all-NaN output (the Frobenius norm is
Inf or NaN, and the products spread it); so does the reference's gram form,
whose norm and products are the same. The library must do the same for the
matrix that holds it, and must leave every other matrix of the same grouped
call exactly as a call without it would compute it (each matrix's stages are
independent, whatever tiles share a launch).
"""
import pytest
import torch

from pan2_amd import _lib
from tests.conftest import TORCH_ZEROPOWER

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
COEFFS = (3.4445, -4.7750, 2.0315)
# engine (short side > 128) wide and tall; small-matrix path wide, tall and a full QKV row block
SHAPES = [(256, 512), (640, 300), (100, 700), (4096, 128)]


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g)


@pytest.mark.parametrize("form", ["standard", "gram"])
@pytest.mark.parametrize("bad", [float("inf"), float("-inf"), float("nan")])
@pytest.mark.parametrize("shape", SHAPES)
def test_nonfinite_input_gives_all_nan(shape, bad, form):
    print(f"nonfinite {shape} {bad} {form}", flush=True)
    x = seeded(shape, 11)
    x[shape[0] // 3, shape[1] // 2] = bad
    want = TORCH_ZEROPOWER(x.bfloat16(), COEFFS, 5, 1e-7)  # torch's own NS, whatever is patched
    assert torch.isnan(want.float()).all()  # torch's own behaviour, on the CPU
    o = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    _lib.newton_schulz_into([(x.to(DEV), o)], ns_form=form)
    assert torch.isnan(o.float()).all()


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_nonfinite_matrix_leaves_its_group_untouched(form):
    """One call over matrices of both paths, one of them holding an Inf and
    another a NaN: those two come out all NaN, every other one bit-identical to
    the same call on all-finite inputs."""
    shapes = [(256, 512), (512, 256), (100, 700), (128, 1024), (300, 640), (96, 384)]
    xs = [seeded(s, 20 + i).to(DEV) for i, s in enumerate(shapes)]
    clean = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, clean)), ns_form=form)
    bad = {1: float("inf"), 3: float("nan")}
    for i, v in bad.items():
        xs[i][5, 9] = v
    got = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, got)), ns_form=form)
    for i in range(len(shapes)):
        if i in bad:
            assert torch.isnan(got[i].float()).all(), i
        else:
            assert torch.equal(got[i], clean[i]), i


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_nonfinite_matrix_in_a_fused_small_group(form):
    """300 small matrices in one call (enough for the fused grams of the
    small-matrix path), one holding a NaN and one an Inf: those come out all NaN,
    the other 298 bit-identical to the call on all-finite inputs."""
    shapes = [(128, 256 + 64 * (i % 5)) for i in range(300)]
    xs = [seeded(s, 100 + i).to(DEV) for i, s in enumerate(shapes)]
    clean = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, clean)), ns_form=form)
    bad = {7: float("nan"), 201: float("-inf")}
    for i, v in bad.items():
        xs[i][60, 100] = v
    got = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, got)), ns_form=form)
    for i in range(len(shapes)):
        if i in bad:
            assert torch.isnan(got[i].float()).all(), i
        else:
            assert torch.equal(got[i], clean[i]), i


@pytest.mark.parametrize("form", ["standard", "gram"])
def test_nonfinite_through_k_split_stages(form):
    """Matrices whose stages run K-split (fp32 chunk partials, then the
    reduce launch; in this call the grams of the 2048 x 2048 and 1024 x 4096
    matrices and the 2048 x 2048 symmetric products split), one holding a NaN and one an Inf, beside finite split and
    unsplit matrices:
    the two come out all NaN (the same products spread it as in the shapes
    above, where torch's NS is checked), the rest bit-identical to the
    all-finite call."""
    shapes = [(2048, 2048), (1024, 4096), (4096, 1024), (2048, 2048), (512, 768)]
    xs = [seeded(s, 40 + i).to(DEV) for i, s in enumerate(shapes)]
    clean = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, clean)), ns_form=form)
    bad = {0: float("nan"), 2: float("inf")}
    for i, v in bad.items():
        xs[i][700, 300] = v
    got = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    _lib.newton_schulz_into(list(zip(xs, got)), ns_form=form)
    for i in range(len(shapes)):
        if i in bad:
            assert torch.isnan(got[i].float()).all(), i
        else:
            assert torch.equal(got[i], clean[i]), i
