"""The drop-in step on a side stream, as PAN 2's validated eager mode runs it.

PAN 2 runs forward, backward and both optimizer steps on a side stream
(train.py:1025-1031). The current stream waits for that stream before the
lr schedulers step (train.py:1039-1044). Every libpanmuon launch and
descriptor upload must go on the caller's current stream, ordered after the
work that produced the grads. So here each step's grads are written on the
side stream behind a GPU spin (torch.cuda._sleep). A step that ran on any
other stream would read the previous grads. Three steps with a
LambdaLR schedule must give the bits of the same steps on the default stream.
PAN 2 creates its side stream with priority 4. Streams here keep the default
priority, which is the only one used on this hardware pool.
"""
import importlib

import pytest
import torch

import torch.optim._muon as torch_muon
from pan2_amd.optim.muon import build_native_muon_optimizers
from tests.test_gpu_state_dict import Block

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ADAM_MODULE = importlib.import_module("torch.optim.adam")
SPIN = 50_000_000  # GPU cycles of torch.cuda._sleep before each step's grads (about 20-30 ms)


@pytest.fixture
def restore_torch_optim():
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, ADAM_MODULE._fused_adam)
    yield
    torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, ADAM_MODULE._fused_adam = saved


def run(side: bool, steps=3):
    model = Block(11).to(DEV)
    opts = build_native_muon_optimizers(model, lr=torch.tensor(0.02, device=DEV), weight_decay=0.01,
                                        capturable=True, muon_chunks={"qkv": (0, 6)})["optimizers"]
    scheds = [torch.optim.lr_scheduler.LambdaLR(o, lambda k: 1.0 / (1 + k)) for o in opts.values()]
    # every step's grads, made on the host beforehand
    host = []
    for k in range(steps):
        g = torch.Generator("cpu").manual_seed(300 + k)
        host.append([(torch.randn(p.shape, generator=g) * 1e-3).pin_memory() for p in model.parameters()])
    for p in model.parameters():
        p.grad = torch.zeros_like(p)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=DEV) if side else torch.cuda.current_stream(DEV)
    for k in range(steps):
        stream.wait_stream(torch.cuda.current_stream(DEV))
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN)  # the side stream is busy: the grads land late
            for p, g in zip(model.parameters(), host[k]):
                p.grad.copy_(g, non_blocking=True)
            for o in opts.values():
                o.step()
        torch.cuda.current_stream(DEV).wait_stream(stream)
        for s in scheds:
            s.step()
    torch.cuda.synchronize()
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    state = {(name, n, key): v.detach().clone()
             for name, o in opts.items() for n, p in model.named_parameters()
             for key, v in o.state.get(p, {}).items()}
    return params, state


def test_step_on_a_side_stream_matches_the_default_stream(restore_torch_optim):
    ref_p, ref_s = run(side=False)
    got_p, got_s = run(side=True)
    assert ref_p.keys() == got_p.keys() and ref_s.keys() == got_s.keys()
    for n in ref_p:
        assert torch.equal(got_p[n], ref_p[n]), n
    for key in ref_s:
        assert torch.equal(got_s[key], ref_s[key]), key
    assert not torch.equal(ref_p["proj"], Block(11).to(DEV).proj.detach())
