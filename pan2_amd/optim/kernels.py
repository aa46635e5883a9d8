"""The public ops of pan/optim/muon_triton.py with the reference's Python
signatures, on libpanmuon.

Drop-ins for ``muon_momentum_nesterov`` (:54-108), ``step_param``
(:164-210), ``can_use_fused_gram_ns`` (:303-312) and
``batched_gram_newtonschulz`` (:315-345). The fused Muon step does not call
these (its prologue, small-matrix kernels and final GEMM epilogue do the same
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


def can_use_fused_gram_ns(x) -> bool:
    """The reference's test for its fused batched gram path
    (pan/optim/muon_triton.py:303-312): a device batch [B >= 96, 128, N >= 128].
    libpanmuon runs any matrix with a short side <= 128 on its small-matrix
    kernels; this keeps the reference's answer for callers that branch on it."""
    return (isinstance(x, torch.Tensor) and x.is_cuda and x.ndim == 3 and x.size(0) >= 96 and x.size(-2) == 128
            and x.size(-1) >= 128)


def batched_gram_newtonschulz(X, ns_coefficients, ns_steps, eps, reset_iterations=frozenset([2])):
    """PAN 2's gram-form Newton–Schulz over a batch X = [B, 128, N]
    (pan/optim/muon_triton.py:315-345, the fused equivalent of
    _gram_newtonschulz_local): returns the orthogonalised bf16 batch. As in the
    reference, a batch that resets at iteration 2 comes back in X's own
    (bf16) storage; libpanmuon's gram form resets at iteration 2 whenever
    ns_steps > 2 (pan/optim/patch_muon.py:286), so other reset sets raise."""
    X = X.to(torch.bfloat16) if X.dtype != torch.bfloat16 else X
    assert X.is_contiguous(), "batched_gram_newtonschulz requires a contiguous [B, 128, N] input"
    assert len(reset_iterations) <= 1, "fused gram-NS supports at most one reset iteration"
    resets = set(reset_iterations)
    if ns_steps > 2 and resets != {2}:
        raise ValueError(f"libpanmuon's gram form resets at iteration 2 for ns_steps > 2; got {sorted(resets)}")
    if ns_steps <= 2 and resets - {2}:
        raise ValueError(f"libpanmuon's gram form does not reset for ns_steps <= 2; got {sorted(resets)}")
    if X.ndim != 3:
        raise ValueError(f"batched_gram_newtonschulz takes [B, M, N], got shape {tuple(X.shape)}")
    if not X.is_cuda:
        raise RuntimeError("pan2_amd Newton–Schulz runs on HIP device tensors only")
    # the reference writes the result back into X when the batch reset (its
    # second segment ran), else returns a new tensor
    out = X if ns_steps > 2 else torch.empty_like(X)
    _lib.newton_schulz_into([(X[i], out[i]) for i in range(X.shape[0])], ns_coefficients=ns_coefficients,
                            ns_steps=ns_steps, eps=eps, ns_form="gram")
    return out
