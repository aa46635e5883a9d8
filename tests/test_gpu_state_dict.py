"""Optimizer state of the drop-in Muon step: the reference's checkpoint
bundle round-trips, and a restored optimizer continues bit-identically.

PAN 2 saves {"format_version": 2, "optimizers": {name: opt.state_dict()}} with
torch.save and restores it with load_state_dict after torch.load(map_location
="cpu") (train.py:1100-1101, 1199-1204). DCP's optimizer-state init runs one
step with the lr swapped for a CPU tensor(0.0) and zero grads (the case
pan/optim/muon_triton.py:182-186 handles). pan2_amd keeps torch's own
optimizer classes, so the state layout is torch's: this pins that it stays so
through the HIP step (momentum_buffer per param, the chunked group's
(base, dim, n_chunks) adjust_lr_fn tuple) and that a restored step matches.
"""
import io

import pytest
import torch

import torch.optim._muon as torch_muon
from pan2_amd.optim.muon import build_native_muon_optimizers

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture
def restore_torch_muon():
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
    yield
    torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = saved


class Block(torch.nn.Module):
    def __init__(self, seed):
        super().__init__()
        g = torch.Generator("cpu").manual_seed(seed)
        self.qkv = torch.nn.Parameter(torch.randn(768, 256, generator=g) * 0.02)    # chunked: 6 x 128 rows
        self.proj = torch.nn.Parameter(torch.randn(256, 512, generator=g) * 0.02)
        self.norm = torch.nn.Parameter(torch.ones(256))                              # AdamW (1-D)
        self.pos_embed = torch.nn.Parameter(torch.randn(64, 256, generator=g) * 0.02)  # AdamW (by name)


def make(seed=7):
    model = Block(seed).to(DEV)
    built = build_native_muon_optimizers(model, lr=torch.tensor(0.02, device=DEV), weight_decay=0.01,
                                         muon_chunks={"qkv": (0, 6)})
    return model, built["optimizers"]


def set_grads(model, step):
    g = torch.Generator("cpu").manual_seed(100 + step)
    for p in model.parameters():
        p.grad = (torch.randn(p.shape, generator=g) * 1e-3).to(DEV)


def step_all(model, opts, step):
    set_grads(model, step)
    for opt in opts.values():
        opt.step()


def test_bundle_round_trip_continues_bit_identically(restore_torch_muon, tmp_path):
    print("state_dict bundle round trip", flush=True)
    model, opts = make()
    step_all(model, opts, 0)
    bundle = {"format_version": 2, "optimizers": {name: opt.state_dict() for name, opt in opts.items()}}
    path = tmp_path / "optimizer_state.pt"
    torch.save(bundle, path)

    # the saved layout is torch's: a momentum_buffer per Muon param, the chunked group's tuple
    muon_sd = bundle["optimizers"]["muon"]
    assert set(muon_sd) == {"state", "param_groups"}
    assert all(set(s) == {"momentum_buffer"} for s in muon_sd["state"].values())
    assert [g["adjust_lr_fn"] for g in muon_sd["param_groups"]] == ["match_rms_adamw", ("match_rms_adamw", 0, 6)]

    # restore into a fresh model holding the same weights, then step both with the same grads
    twin, twin_opts = make(seed=999)
    with torch.no_grad():
        for a, b in zip(twin.parameters(), model.parameters()):
            a.copy_(b)
    saved = torch.load(path, map_location="cpu", weights_only=True)
    assert saved["format_version"] == 2
    for name, opt in twin_opts.items():
        opt.load_state_dict(saved["optimizers"][name])
    assert twin_opts["muon"].param_groups[1]["adjust_lr_fn"] == ("match_rms_adamw", 0, 6)
    # torch restores the saved group values as they are, so a tensor lr comes back on the CPU;
    # PAN 2 refuses to train on a CPU-tensor lr after a load (train.py:1216-1225), so the
    # resumed run puts it back on the device, where the step reads it
    for opt in twin_opts.values():
        for g in opt.param_groups:
            assert isinstance(g["lr"], torch.Tensor) and g["lr"].device.type == "cpu"
            assert g["lr"].item() == pytest.approx(0.02)
            g["lr"] = g["lr"].to(DEV)
    for s in twin_opts["muon"].state.values():
        assert s["momentum_buffer"].is_cuda and s["momentum_buffer"].dtype == torch.float32

    step_all(model, opts, 1)
    step_all(twin, twin_opts, 1)
    torch.cuda.synchronize()
    for (n, a), b in zip(model.named_parameters(), twin.parameters()):
        assert torch.equal(a, b), n
    for pa, pb in zip(opts["muon"].state.values(), twin_opts["muon"].state.values()):
        assert torch.equal(pa["momentum_buffer"], pb["momentum_buffer"])


def test_dcp_style_zero_lr_dummy_step(restore_torch_muon):
    """lr swapped for a CPU tensor(0.0) and zero grads: the state is created,
    params and momentum stay as they were (all zeros in, zeros out)."""
    print("zero-lr cpu-tensor dummy step", flush=True)
    model, opts = make()
    muon = opts["muon"]
    before = [p.detach().clone() for p in model.parameters()]
    saved_lrs = [g["lr"] for g in muon.param_groups]
    for g in muon.param_groups:
        g["lr"] = torch.tensor(0.0)
    for p in model.parameters():
        p.grad = torch.zeros_like(p)
    muon.step()
    torch.cuda.synchronize()
    muon_params = {id(p) for g in muon.param_groups for p in g["params"]}
    for p, b in zip(model.parameters(), before):
        if id(p) in muon_params:
            assert torch.equal(p, b)
            assert torch.count_nonzero(muon.state[p]["momentum_buffer"]).item() == 0
    for g, lr in zip(muon.param_groups, saved_lrs):
        g["lr"] = lr
    step_all(model, opts, 2)  # a normal step still runs after the swap back
    torch.cuda.synchronize()
