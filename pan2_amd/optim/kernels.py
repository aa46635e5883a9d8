"""Elementwise Muon ops with the reference's Python signatures, on libpanmuon.

Drop-ins for the two elementwise entry points of pan/optim/muon_triton.py:
``muon_momentum_nesterov`` (:54-108) and ``step_param`` (:164-210). The fused
Muon step does not call these (its prologue and final GEMM epilogue do the same
arithmetic); they exist for callers that use the reference's module directly.
"""
from __future__ import annotations

import torch

from .. import _lib
from .patch_muon import _adjust_ratio


def muon_momentum_nesterov(buf, grad, momentum: float, output_dtype=None, out=None):
    """buf <- mu*buf + (1-mu)*g (in place); returns u = (1-mu)*g + mu*buf.

    Same contract as pan/optim/muon_triton.py:54-108: ``out`` and
    ``output_dtype`` are exclusive; ``out`` receives the update in place.
    """
    assert out is None or output_dtype is None, "`out` and `output_dtype` cannot both be passed"
    assert buf.shape == grad.shape, "buf and grad must have the same shape"
    assert buf.is_contiguous() and grad.is_contiguous(), "buf and grad must be contiguous"
    if out is not None:
        assert out.shape == grad.shape, "out must have the same (local) shape as grad"
        assert out.is_contiguous(), "out must be contiguous"
        update = out
    else:
        update = torch.empty(grad.shape, dtype=output_dtype or grad.dtype, device=grad.device)
    _lib.momentum_nesterov_into(buf, grad, update, momentum, nesterov=True)
    return update


def step_param(param, update, lr, weight_decay, base_adjust_lr_fn, shape) -> None:
    """p <- p*(1 - lr*wd) - adjusted_lr*u in place (pan/optim/muon_triton.py:164-210).

    lr may be a float, a device 0-d tensor (read on the device) or a CPU 0-d
    tensor (taken as a host scalar, :182-186).
    """
    assert param.shape == update.shape, "param and update must have the same shape"
    assert param.is_contiguous() and update.is_contiguous(), "param and update must be contiguous"
    _lib.step_param_inplace(param, update, lr, weight_decay, _adjust_ratio(base_adjust_lr_fn, shape))
