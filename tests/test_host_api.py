"""Host-side drop-in API (pan2_amd.optim) on the CPU: parameter split, factory
groups, patch installation, argument errors and the host-side LR scheduler,
against the reference's behaviour (pan/optim/muon.py, patch_muon.py,
patch_lr_scheduler.py). No device work."""
import pytest
import torch
import torch.optim._muon as torch_muon

from pan2_amd.optim import patch_muon as pm
from pan2_amd.optim.kernels import muon_momentum_nesterov
from pan2_amd.optim.muon import (_looks_like_embedding_or_head, build_native_muon_optimizers,
                                 split_params_for_native_muon)
from pan2_amd.optim.patch_lr_scheduler import patch_lr_scheduler


class Tiny(torch.nn.Module):
    """Names cover every exclusion rule of pan/optim/muon.py:24-50."""

    def __init__(self):
        super().__init__()
        self.embed_tokens = torch.nn.Embedding(10, 8)
        self.patch_embed = torch.nn.Linear(8, 8)
        self.timestep_encoder = torch.nn.Linear(8, 8)
        self.blocks = torch.nn.ModuleList([torch.nn.ModuleDict({
            "attn": torch.nn.Linear(8, 16),
            "mlp": torch.nn.Linear(16, 8, bias=False),
            "modulation": torch.nn.ModuleDict({"lin": torch.nn.Linear(8, 48)}),
            "norm": torch.nn.LayerNorm(8),
        })])
        self.lm_head = torch.nn.Linear(8, 10)
        self.frozen = torch.nn.Linear(8, 8)
        self.frozen.requires_grad_(False)


@pytest.fixture
def restore_torch_muon():
    from torch.optim.lr_scheduler import LambdaLR

    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, LambdaLR.get_last_lr,
             LambdaLR.__init__, LambdaLR.load_state_dict)
    yield
    (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, LambdaLR.get_last_lr,
     LambdaLR.__init__, LambdaLR.load_state_dict) = saved


def test_exclusion_rules():
    for name in ("embed_tokens.weight", "model.pos_embed", "lm_head.weight", "blocks.0.modulation.lin.weight",
                 "text_modulation.weight", "timestep_encoder.0.weight", "patch_embed.proj.weight",
                 "output_head.weight", "x.classifier.weight", "Token_Embed.w"):
        assert _looks_like_embedding_or_head(name), name
    for name in ("blocks.0.attn.weight", "blocks.0.mlp.weight", "decoder.out_proj.weight", "my_patch_embed.w"):
        assert not _looks_like_embedding_or_head(name), name


def test_split_params():
    model = Tiny()
    muon, adamw, stats = split_params_for_native_muon(model)
    assert [n for n, _ in muon] == ["blocks.0.attn.weight", "blocks.0.mlp.weight"]
    names = {n for n, _ in adamw}
    assert "blocks.0.attn.bias" in names and "lm_head.weight" in names and "frozen.weight" not in names
    assert stats["muon_param_tensors"] == 2
    assert stats["muon_param_numel"] == 8 * 16 + 16 * 8
    assert stats["trainable_param_tensors"] == len(muon) + len(adamw)
    # 2-D weights kept on AdamW by name: embedding, patch_embed, timestep, modulation, lm_head
    assert stats["excluded_embedding_or_head_tensors"] == 5


def test_factory_float_lr_keeps_stock_torch(restore_torch_muon):
    before = torch_muon._single_tensor_muon
    out = build_native_muon_optimizers(Tiny(), lr=1e-3, weight_decay=0.05)
    assert torch_muon._single_tensor_muon is before, "a float lr must not patch (pan/optim/muon.py:126-128)"
    muon = out["optimizers"]["muon"]
    assert isinstance(muon, torch.optim.Muon)
    assert muon.defaults["adjust_lr_fn"] == "match_rms_adamw" and muon.defaults["momentum"] == 0.95
    assert muon.defaults["weight_decay"] == 0.05
    adamw = out["optimizers"]["adamw"]
    assert isinstance(adamw, torch.optim.AdamW) and adamw.defaults["fused"]
    assert adamw.defaults["betas"] == (0.95, 0.95)
    assert out["param_names"]["muon_chunked"] == []


def test_factory_chunk_groups_and_tensor_lr(restore_torch_muon):
    model = Tiny()
    lr = torch.tensor(2e-3)
    out = build_native_muon_optimizers(model, lr=lr, muon_chunks={"blocks.0.attn.weight": (0, 2)})
    assert torch_muon._single_tensor_muon is pm._single_tensor_muon
    assert torch_muon._zeropower_via_newtonschulz is pm.newton_schulz
    muon = out["optimizers"]["muon"]
    assert len(muon.param_groups) == 2
    assert muon.param_groups[1]["adjust_lr_fn"] == ("match_rms_adamw", 0, 2)
    assert muon.param_groups[1]["params"][0] is model.blocks[0]["attn"].weight
    assert out["param_names"]["muon_chunked"] == [("blocks.0.attn.weight", 0, 2)]
    assert out["param_names"]["muon"] == ["blocks.0.mlp.weight"]
    # the optimizer holds a clone of the tensor lr, not the caller's tensor
    assert muon.param_groups[0]["lr"] is not lr and float(muon.param_groups[0]["lr"]) == pytest.approx(2e-3)


def test_factory_without_trainable_params():
    m = torch.nn.Linear(4, 4)
    m.requires_grad_(False)
    with pytest.raises(ValueError, match="No trainable parameters"):
        build_native_muon_optimizers(m)


def _call(params, grads, bufs, **kw):
    args = dict(lr=0.02, weight_decay=0.0, momentum=0.95, nesterov=True, ns_coefficients=(3.4445, -4.775, 2.0315),
                ns_steps=5, eps=1e-7, adjust_lr_fn=None, has_complex=False)
    args.update(kw)
    return pm._single_tensor_muon(params, grads, bufs, **args)


def test_single_tensor_muon_argument_errors():
    z = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        _call([torch.zeros(8)], [torch.zeros(8)], [torch.zeros(8)])
    with pytest.raises(ValueError, match="complex"):
        _call([z], [z], [z], has_complex=True)
    with pytest.raises(AssertionError, match="dim 1"):
        _call([z], [z], [z], adjust_lr_fn=("match_rms_adamw", 1, 2))
    with pytest.raises(AssertionError):
        _call([z], [z], [z], nesterov=False)
    with pytest.raises(AssertionError, match="divisible"):
        _call([torch.zeros(5, 8)], [torch.zeros(5, 8)], [torch.zeros(5, 8)], adjust_lr_fn=("match_rms_adamw", 0, 2))
    assert _call([], [], []) is None


def test_adjust_ratio_and_scalar_lr():
    assert pm._adjust_ratio(None, (4096, 1024)) == 2.0
    assert pm._adjust_ratio("match_rms_adamw", (256, 1024)) == pytest.approx(6.4)
    assert pm._scalar_lr(torch.tensor([0.5])).ndim == 0
    assert pm._scalar_lr(0.5) == 0.5


def test_newton_schulz_argument_errors():
    with pytest.raises(ValueError, match="less than 100"):
        pm.newton_schulz(torch.zeros(4, 4), (3.4445, -4.775, 2.0315), 100, 1e-7)
    with pytest.raises(ValueError, match="2D"):
        pm.newton_schulz(torch.zeros(4), (3.4445, -4.775, 2.0315), 5, 1e-7)


def test_momentum_out_and_dtype_exclusive():
    z = torch.zeros(4)
    with pytest.raises(AssertionError, match="cannot both"):
        muon_momentum_nesterov(z, z, 0.9, output_dtype=torch.bfloat16, out=z)


def test_lr_scheduler_host_get_last_lr(restore_torch_muon):
    from torch.optim.lr_scheduler import LambdaLR

    p = torch.nn.Parameter(torch.zeros(2, 2))
    opt = torch.optim.SGD([p], lr=torch.tensor(0.1))
    sched = LambdaLR(opt, lambda e: 0.5 ** e)
    patch_lr_scheduler()
    for epoch in range(3):
        got = sched.get_last_lr()
        assert all(isinstance(v, float) for v in got)
        assert got == [pytest.approx(0.1 * 0.5 ** epoch)]
        opt.step()
        sched.step()
    # load_state_dict re-reads the base learning rates
    other = LambdaLR(torch.optim.SGD([torch.nn.Parameter(torch.zeros(1))], lr=torch.tensor(0.4)), lambda e: 0.5 ** e)
    sched.load_state_dict(other.state_dict())
    assert sched.get_last_lr() == [pytest.approx(0.4 * 0.5 ** sched.last_epoch)]


def test_lr_scheduler_reads_base_lrs_only_at_capture(restore_torch_muon):
    """A LambdaLR built after the patch reads its base learning rates once, when
    it is constructed: get_last_lr() never touches them again, and the host
    copy stays out of state_dict()."""
    from torch.optim.lr_scheduler import LambdaLR

    reads = []

    class Counted(float):
        """A base lr that records every host read (float()) of itself."""

        def __float__(self):
            reads.append(1)
            return super().__float__()

    patch_lr_scheduler()
    patch_lr_scheduler()  # idempotent
    opt = torch.optim.SGD([torch.nn.Parameter(torch.zeros(2))], lr=Counted(0.3))
    sched = LambdaLR(opt, [lambda e: 1.0 / (e + 1)])
    assert reads == [1]
    sd_keys = set(sched.state_dict())
    for epoch in range(3):
        assert sched.get_last_lr() == [pytest.approx(0.3 / (epoch + 1))]
        opt.step()
        sched.step()
    assert reads == [1]
    assert not any("host" in k or "pan2" in k for k in sd_keys)


def test_lr_scheduler_base_lrs_assignment_recaptured(restore_torch_muon):
    """Assigning a new base_lrs list (outside load_state_dict) is picked up by
    the next get_last_lr(), with one read per base lr; an unchanged list is
    not read again (pan/optim/patch_lr_scheduler.py:23 re-reads on list
    identity)."""
    from torch.optim.lr_scheduler import LambdaLR

    reads = []

    class Counted(float):
        def __float__(self):
            reads.append(1)
            return super().__float__()

    patch_lr_scheduler()
    opt = torch.optim.SGD([torch.nn.Parameter(torch.zeros(2))], lr=0.3)
    sched = LambdaLR(opt, lambda e: 0.5 ** e)
    assert sched.get_last_lr() == [pytest.approx(0.3)]
    sched.base_lrs = [Counted(0.8)]
    assert sched.get_last_lr() == [pytest.approx(0.8)]
    assert reads == [1]
    opt.step()
    sched.step()
    assert sched.get_last_lr() == [pytest.approx(0.8 * 0.5)]
    assert reads == [1]


def test_adam_descriptor_pass_layout_and_statuses():
    """_pm_host.fill_adam (pan2_amd/csrc/pm_host.cpp) on CPU tensors (hip_only
    off): every field of the pm_adam_tensor array _lib hands to pm_adam_step,
    read back through the ctypes layout; and the statuses the AdamW path
    branches on."""
    import ctypes

    import numpy as np

    from pan2_amd import _lib

    h = _lib.host_ext()
    assert h.DESC_BYTES == ctypes.sizeof(_lib.PmAdamTensor) == 72
    dts = [torch.float32, torch.bfloat16, torch.float16]
    ps = [torch.zeros(5 + 3 * i, dtype=dts[i % 3]) for i in range(7)]
    gs = [torch.zeros(p.shape, dtype=dts[(i + 1) % 3]) for i, p in enumerate(ps)]
    ms = [torch.zeros(p.shape, dtype=dts[(i + 2) % 3]) for i, p in enumerate(ps)]
    vs = [torch.zeros(p.shape, dtype=dts[i % 3]) for i, p in enumerate(ps)]
    xs = [torch.zeros_like(v) for v in vs]
    st = [torch.zeros((), dtype=torch.float32) for _ in ps]
    for ams in (False, True):
        arr = np.zeros(len(ps), dtype=_lib._PM_ADAM_NP)
        assert h.fill_adam(arr.ctypes.data, ps, gs, ms, vs, xs if ams else [], st, hip_only=False) == h.FILLED
        c = (_lib.PmAdamTensor * len(ps)).from_address(arr.ctypes.data)
        for i in range(len(ps)):
            assert (c[i].param, c[i].grad, c[i].exp_avg, c[i].exp_avg_sq, c[i].step) == (
                ps[i].data_ptr(), gs[i].data_ptr(), ms[i].data_ptr(), vs[i].data_ptr(), st[i].data_ptr())
            assert (c[i].max_exp_avg_sq or 0) == (xs[i].data_ptr() if ams else 0)
            assert c[i].numel == ps[i].numel()
            assert [c[i].param_dtype, c[i].grad_dtype, c[i].exp_avg_dtype, c[i].exp_avg_sq_dtype] == [
                _lib.adam_dtype_code(t) for t in (ps[i], gs[i], ms[i], vs[i])]
    arr = np.zeros(len(ps), dtype=_lib._PM_ADAM_NP)
    # the product path takes HIP tensors only: CPU lists are the general path's
    assert h.fill_adam(arr.ctypes.data, ps, gs, ms, vs, [], st) == h.GENERAL
    assert _lib.adam_descs(ps, gs, ms, vs, [], st) is None
    # a dtype pm_adam_step does not take, float64 steps, a max_exp_avg_sq of another dtype
    for bad in ({"p": torch.zeros(4, dtype=torch.float64)}, {"s": torch.zeros((), dtype=torch.float64)},
                {"x": torch.zeros(ps[0].shape, dtype=torch.float64)}):
        p2, s2, x2 = [bad.get("p", ps[0])] + ps[1:], [bad.get("s", st[0])] + st[1:], [bad.get("x", xs[0])] + xs[1:]
        assert h.fill_adam(arr.ctypes.data, p2, gs, ms, vs, x2 if "x" in bad else [], s2, hip_only=False) == h.GENERAL
    # pm_adam_step walks the tensors as flat arrays of the param's length: a
    # tensor that is not contiguous (here a strided grad, a transposed param
    # with state of its strides, a strided max_exp_avg_sq) or of another
    # element count goes to the general path
    p43 = torch.zeros(4, 3)
    assert h.fill_adam(arr.ctypes.data, [p43] + ps[1:], [torch.zeros(4, 6)[:, ::2]] + gs[1:], ms, vs, [], st,
                       hip_only=False) == h.GENERAL
    pt = torch.zeros(3, 4).t()
    assert h.fill_adam(arr.ctypes.data, [pt] + ps[1:], [torch.zeros_like(pt)] + gs[1:], [torch.zeros_like(pt)] + ms[1:],
                       [torch.zeros_like(pt)] + vs[1:], [], st, hip_only=False) == h.GENERAL
    assert h.fill_adam(arr.ctypes.data, ps, gs, ms, vs, [torch.zeros(2 * ps[0].numel())[::2]] + xs[1:], st,
                       hip_only=False) == h.GENERAL
    for short in ("g", "m", "v", "x"):
        t = torch.zeros(ps[0].numel() - 1, dtype=ps[0].dtype)
        lists = {k: list(v) for k, v in (("g", gs), ("m", ms), ("v", vs), ("x", xs))}
        lists[short][0] = t
        assert h.fill_adam(arr.ctypes.data, ps, lists["g"], lists["m"], lists["v"], lists["x"], st,
                           hip_only=False) == h.GENERAL, short
    assert h.fill_adam(arr.ctypes.data, ps, gs, ms, vs, [], [torch.zeros(2)] + st[1:], hip_only=False) == h.GENERAL
    with pytest.raises(RuntimeError, match="differ in length"):
        h.fill_adam(arr.ctypes.data, ps, gs[:-1], ms, vs, [], st, hip_only=False)
    assert h.fill_adam(0, [], [], [], [], [], []) == h.FILLED


def test_fused_gram_ns_predicate_and_reset_sets():
    """pan/optim/muon_triton.py:303-345's public pair, on the host: the
    predicate keeps the reference's answer, and reset sets the library's gram
    form does not run raise before anything else."""
    from pan2_amd.optim.kernels import batched_gram_newtonschulz, can_use_fused_gram_ns

    assert not can_use_fused_gram_ns(torch.zeros(96, 128, 256))  # a CPU tensor
    assert not can_use_fused_gram_ns(torch.zeros(128, 256)) and not can_use_fused_gram_ns(None)
    x = torch.zeros(4, 128, 256)
    with pytest.raises(ValueError, match="iteration 2"):
        batched_gram_newtonschulz(x, (3.4445, -4.7750, 2.0315), 5, 1e-7, reset_iterations=frozenset([3]))
    with pytest.raises(ValueError, match="iteration 2"):
        batched_gram_newtonschulz(x, (3.4445, -4.7750, 2.0315), 5, 1e-7, reset_iterations=frozenset())
    with pytest.raises(ValueError, match="does not reset"):
        batched_gram_newtonschulz(x, (3.4445, -4.7750, 2.0315), 2, 1e-7, reset_iterations=frozenset([1]))
    with pytest.raises(RuntimeError, match="HIP device"):
        batched_gram_newtonschulz(x, (3.4445, -4.7750, 2.0315), 5, 1e-7)
