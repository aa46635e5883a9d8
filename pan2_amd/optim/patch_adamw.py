"""The AdamW half of PAN 2's optimizer step on MI355X, installed over torch's
fused Adam by :func:`patch_adamw`.

PAN 2 builds ``torch.optim.AdamW(fused=True)`` over the params Muon does not
take (pan/optim/muon.py:155-164). ``AdamW.step`` reaches the module-global
``_fused_adam`` of the torch.optim.adam module (TORCH/optim/adam.py:963-964,
:803-898);
:func:`patch_adamw` replaces it with a keyword-compatible function that hands
every tensor of the group to libpanmuon's ``pm_adam_step`` in one call: the
step counts and the element update run as two HIP launches on the current
stream, with no host synchronisation. The optimizer object, its param groups
and its state (``step``, ``exp_avg``, ``exp_avg_sq``) stay torch's, so
state_dict and checkpoints are unchanged.

Tensors the library does not take (float64, complex, on the CPU, or not
contiguous) go to torch's own fused Adam, saved when this module is imported,
exactly as an unpatched process would run them; contiguous fp32, bf16 and fp16
device tensors go to ``pm_adam_step``.
"""
from __future__ import annotations

import importlib

import torch
from torch import Tensor

from .. import _lib

# torch.optim does not keep its adam submodule as an attribute
_adam_module = importlib.import_module("torch.optim.adam")
# torch's own fused Adam, for the tensors pm_adam_step does not take
_torch_fused_adam = _adam_module._fused_adam


def _scalar(x):
    """A 1-element tensor beta becomes a Python float (torch's _to_scalar)."""
    return x.item() if isinstance(x, Tensor) else x


def _native(i, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, amsgrad) -> bool:
    """Does pm_adam_step take tensor i: contiguous fp32 / bf16 / fp16 device
    tensors of the param's size throughout? (It walks them as flat arrays.)"""
    ts = [params[i], grads[i], exp_avgs[i], exp_avg_sqs[i]] + ([max_exp_avg_sqs[i]] if amsgrad else [])
    n = params[i].numel()
    return all(t.is_cuda and t.dtype in _lib.ADAM_DTYPES and t.is_contiguous() and t.numel() == n for t in ts)


@torch.compiler.disable
def _fused_adam(
    params: list[Tensor],
    grads: list[Tensor],
    exp_avgs: list[Tensor],
    exp_avg_sqs: list[Tensor],
    max_exp_avg_sqs: list[Tensor],
    state_steps: list[Tensor],
    grad_scale: Tensor | None,
    found_inf: Tensor | None,
    *,
    amsgrad: bool,
    has_complex: bool,
    beta1,
    beta2,
    lr,
    weight_decay: float,
    eps: float,
    maximize: bool,
    capturable: bool,
    differentiable: bool,
    decoupled_weight_decay: bool,
) -> None:
    """Keyword-compatible replacement of TORCH/optim/adam.py:803-898 (one call per device)."""
    if not params:
        return
    if differentiable:
        raise RuntimeError("Adam with fused=True does not support differentiable=True")
    beta1, beta2 = _scalar(beta1), _scalar(beta2)
    # The common case, checked and turned into descriptors in one C++ pass:
    # every tensor on params[0]'s HIP device with a dtype pm_adam_step takes.
    arr = None
    if params[0].is_cuda:
        arr = _lib.adam_descs(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs if amsgrad else [],
                              state_steps)
    if arr is not None:
        dev = params[0].device
        dev_lr = lr
        if isinstance(lr, Tensor) and lr.device.type != "cpu" and lr.device != dev:
            dev_lr = lr.to(device=dev, non_blocking=True)
        _lib.adam_launch(
            arr, dev, lr=dev_lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
            maximize=maximize, decoupled=decoupled_weight_decay,
            grad_scale=None if grad_scale is None else grad_scale.to(dev, non_blocking=True),
            found_inf=None if found_inf is None else found_inf.to(dev, non_blocking=True),
        )
        return
    mine = [_native(i, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, amsgrad) for i in range(len(params))]
    if not all(mine):
        rest = [i for i, m in enumerate(mine) if not m]
        pick = lambda xs: [xs[i] for i in rest] if xs else xs  # noqa: E731
        _torch_fused_adam(
            pick(params), pick(grads), pick(exp_avgs), pick(exp_avg_sqs), pick(max_exp_avg_sqs), pick(state_steps),
            grad_scale, found_inf, amsgrad=amsgrad, has_complex=has_complex, beta1=beta1, beta2=beta2, lr=lr,
            weight_decay=weight_decay, eps=eps, maximize=maximize, capturable=capturable,
            differentiable=differentiable, decoupled_weight_decay=decoupled_weight_decay)
        keep = [i for i, m in enumerate(mine) if m]
        if not keep:
            return
        pick = lambda xs: [xs[i] for i in keep] if xs else xs  # noqa: E731
        params, grads, exp_avgs, exp_avg_sqs = pick(params), pick(grads), pick(exp_avgs), pick(exp_avg_sqs)
        max_exp_avg_sqs, state_steps = pick(max_exp_avg_sqs), pick(state_steps)
    by_device: dict[torch.device, list[int]] = {}
    for i, p in enumerate(params):
        by_device.setdefault(p.device, []).append(i)
    for dev, idx in by_device.items():
        pick = lambda xs: [xs[i] for i in idx]  # noqa: E731
        dev_lr = lr
        if isinstance(lr, Tensor) and lr.device.type != "cpu" and lr.device != dev:
            dev_lr = lr.to(device=dev, non_blocking=True)
        _lib.adam_step(
            pick(params), pick(grads), pick(exp_avgs), pick(exp_avg_sqs),
            pick(max_exp_avg_sqs) if amsgrad else [], pick(state_steps),
            lr=dev_lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
            maximize=maximize, decoupled=decoupled_weight_decay,
            grad_scale=None if grad_scale is None else grad_scale.to(dev, non_blocking=True),
            found_inf=None if found_inf is None else found_inf.to(dev, non_blocking=True),
            trusted=True,
        )


def patch_adamw() -> None:
    """Install the HIP path behind every ``fused=True`` Adam / AdamW step.

    Loads libpanmuon and the _pm_host extension first, so a missing or broken
    build fails here, loudly.
    """
    _lib.load()
    _lib.host_ext()
    _adam_module._fused_adam = _fused_adam
