"""PAN 2's compile_optimizer option on the drop-in.

PAN 2 can wrap each optimizer's step in torch.compile(mode="max-autotune-no-
cudagraphs", dynamic=False) (train.py:924-926). It does so in its one validated
mode: a device-tensor lr and capturable AdamW (train.py:853-864, 313). The
HIP entry points are torch.compiler.disable'd, as the reference's
_single_tensor_muon is (pan/optim/patch_muon.py:43). So the compiled step runs
them eagerly between its compiled pieces. Two compiled steps must leave the
params and every optimizer state tensor bit-identical to two eager steps.
Both steps must run on libpanmuon: the launch records count its kernels.
"""
import importlib

import pytest
import torch

import torch.optim._muon as torch_muon
from pan2_amd import _lib
from pan2_amd.optim.muon import build_native_muon_optimizers
from tests.test_gpu_state_dict import Block, set_grads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ADAM_MODULE = importlib.import_module("torch.optim.adam")


@pytest.fixture
def restore_torch_optim():
    saved = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, ADAM_MODULE._fused_adam)
    yield
    torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon, ADAM_MODULE._fused_adam = saved


def run(compiled, steps=2):
    torch._dynamo.reset()
    model = Block(7).to(DEV)
    opts = build_native_muon_optimizers(model, lr=torch.tensor(0.02, device=DEV), weight_decay=0.01,
                                        capturable=True, muon_chunks={"qkv": (0, 6)})["optimizers"]
    assert set(opts) == {"muon", "adamw"}
    if compiled:
        for opt in opts.values():
            opt.step = torch.compile(opt.step, mode="max-autotune-no-cudagraphs", dynamic=False)
    _lib.timing_enable(True)
    try:
        _lib.timing_read()
        for k in range(steps):
            set_grads(model, k)
            for opt in opts.values():
                opt.step()
        torch.cuda.synchronize()
        kinds = [r["kind"] for r in _lib.timing_read()]
    finally:
        _lib.timing_enable(False)
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    state = {}
    for name, opt in opts.items():
        for n, p in model.named_parameters():
            for key, v in opt.state.get(p, {}).items():
                state[(name, n, key)] = v.detach().clone() if isinstance(v, torch.Tensor) else v
    return params, state, kinds


def test_compiled_optimizer_steps_match_eager(restore_torch_optim):
    eager_p, eager_s, eager_k = run(compiled=False)
    comp_p, comp_s, comp_k = run(compiled=True)
    print(f"eager launches {len(eager_k)}, compiled {len(comp_k)}; state tensors {len(eager_s)}", flush=True)
    # Muon (chunked qkv on the small path, proj on the engine) and AdamW ran on libpanmuon in both
    for kinds in (eager_k, comp_k):
        assert kinds.count("adam") == 2 and "small_core" in kinds and "final" in kinds
    assert comp_k == eager_k
    assert eager_p.keys() == comp_p.keys() and eager_s.keys() == comp_s.keys()
    for n in eager_p:
        assert torch.equal(comp_p[n], eager_p[n]), n
    for key in eager_s:
        a, b = eager_s[key], comp_s[key]
        assert (torch.equal(a, b) if isinstance(a, torch.Tensor) else a == b), key
    # the step moved the params
    assert not torch.equal(eager_p["proj"], Block(7).to(DEV).proj.detach())
