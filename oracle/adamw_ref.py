"""numpy restatement of one Adam / AdamW step (test infrastructure only).

Restates ``_single_tensor_adam`` of the third-party torch.optim.adam module
(``TORCH/optim/adam.py:347-549``, torch 2.10 text; the reference pins 2.12.1,
requirements.txt:14), which PAN 2 reaches as ``torch.optim.AdamW(fused=True)``
(pan/optim/muon.py:155-164; fused dispatch TORCH/optim/adam.py:963-964). The
arithmetic is fp32 with the step's scalars formed as torch forms them (Python
doubles rounded to fp32 where they meet a tensor), every operation rounded
once, no fused multiply-adds, and each stored result rounded once to its
storage dtype (fp32 or bf16), as torch's fused kernel stores them.

Pinned in tests/test_oracle.py against torch's own CPU AdamW / Adam (a
library routine: within a few fp32 ulps, torch's vectorised lerp fuses its
multiply-add) and against the closed form of a first step from zero state.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16

f32 = np.float32


def _store(x, dtype: str):
    """The stored value of an fp32 result: "f32" as is, "bf16" or "f16" rounded
    to nearest even (numpy's IEEE half cast for f16)."""
    x = np.asarray(x, dtype=f32)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        with np.errstate(over="ignore"):  # beyond fp16's range: inf, as torch's cast gives
            return x.astype(np.float16).astype(f32)
    return x


def lerp(start, end, w):
    """ATen's scalar lerp: start + w (end - start) if |w| < 0.5, else end - (end - start)(1 - w)."""
    w = f32(w)
    if abs(w) < 0.5:
        return start + w * (end - start)
    return end - (end - start) * (f32(1) - w)


def adam_step(param, grad, exp_avg, exp_avg_sq, step, *, lr: float, beta1: float, beta2: float, eps: float,
              weight_decay: float, decoupled: bool = True, amsgrad: bool = False, max_exp_avg_sq=None,
              maximize: bool = False, grad_scale: float | None = None, dtypes=("f32", "f32", "f32")):
    """One step; returns (param, exp_avg, exp_avg_sq, max_exp_avg_sq, step).

    Arrays hold the values of the stored tensors as float32; dtypes gives the
    storage of (param, exp_avg, exp_avg_sq) ("f32", "bf16" or "f16"). lr, betas, eps
    and weight_decay are Python floats. step is the stored step before this
    call (torch increments it first, TORCH/optim/adam.py:414).
    """
    p = np.asarray(param, dtype=f32)
    g = np.asarray(grad, dtype=f32)
    m = np.asarray(exp_avg, dtype=f32)
    v = np.asarray(exp_avg_sq, dtype=f32)
    step = float(f32(step) + f32(1))                       # :414
    gr = -g if maximize else g                              # :407
    if grad_scale is not None:
        gr = gr / f32(grad_scale)  # (torch's fused kernel also stores the unscaled grad)
    if weight_decay != 0:                                   # :416-429
        if decoupled:
            p = p * f32(1 - lr * weight_decay)
        else:
            gr = gr + f32(weight_decay) * p
    m = lerp(m, gr, 1 - beta1)                              # :457
    v = v * f32(beta2) + (f32(1 - beta2) * gr) * gr         # :476
    bc1 = 1 - beta1 ** step                                 # :531-536, in double
    bc2 = 1 - beta2 ** step
    step_size = lr / bc1
    bc2_sqrt = bc2 ** 0.5
    vmax = None
    vh = v
    if amsgrad:                                             # :539-543
        x = np.asarray(max_exp_avg_sq, dtype=f32)
        vmax = np.where(np.isnan(x) | np.isnan(v), x + v, np.maximum(x, v)).astype(f32)
        vh = vmax
    denom = np.sqrt(vh) / f32(bc2_sqrt) + f32(eps)          # :545
    p = p + f32(-step_size) * (m / denom)                   # :547
    pd, md, vd = dtypes
    return (_store(p, pd), _store(m, md), _store(v, vd), None if vmax is None else _store(vmax, vd), f32(step))
