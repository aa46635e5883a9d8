"""numpy restatement of the Muon step's arithmetic (test infrastructure only).

Each function names the reference lines it restates. ``TORCH`` is the
third-party torch.optim._muon module (torch 2.10 text; the reference pins
2.12.1, requirements.txt:14), whose stock Muon is what the reference runs when
lr is a float (pan/optim/muon.py:126).
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np

from .bf16 import round_bf16

# TORCH/optim/_muon.py:24-28
EPS = 1e-7
DEFAULT_COEFFS = (3.4445, -4.7750, 2.0315)
DEFAULT_NS_STEPS = 5

f32 = np.float32


def adjust_lr_ratio(adjust_lr_fn, shape) -> float:
    """Shape factor of TORCH/optim/_muon.py:73-84 (adjusted_lr = lr * ratio).

    None / "original": sqrt(max(1, A/B)); "match_rms_adamw": 0.2*sqrt(max(A, B));
    anything else: 1. (A, B) = shape[:2].
    """
    A, B = shape[0], shape[1]
    if adjust_lr_fn is None or adjust_lr_fn == "original":
        return math.sqrt(max(1, A / B))
    if adjust_lr_fn == "match_rms_adamw":
        return 0.2 * math.sqrt(max(A, B))
    return 1.0


def momentum_nesterov(buf, grad, momentum: float, nesterov: bool = True):
    """pan/optim/muon_triton.py:41-48 in fp32: returns (new_buf, update).

    new_buf = mu*buf + (1-mu)*g ; update = (1-mu)*g + mu*new_buf (nesterov),
    else update = new_buf (TORCH/optim/_muon.py:311). Each product and sum is
    rounded to fp32 separately (no fused multiply-add).
    """
    mu = f32(momentum)
    omu = f32(1.0) - mu
    b = np.asarray(buf, dtype=np.float32)
    g = np.asarray(grad, dtype=np.float32)
    nb = (mu * b).astype(np.float32) + (omu * g).astype(np.float32)
    nb = nb.astype(np.float32)
    if not nesterov:
        return nb, nb.copy()
    u = ((omu * g).astype(np.float32) + (mu * nb).astype(np.float32)).astype(np.float32)
    return nb, u


def step_factors(lr: float, weight_decay: float, ratio: float):
    """(1 - lr*wd, -lr*ratio) as the reference computes them on the host in
    double and hands them to its fp32 kernel (pan/optim/muon_triton.py:188-190)."""
    return f32(1.0 - lr * weight_decay), f32(-(lr * ratio))


def step_param(param, update, lr: float, weight_decay: float, ratio: float):
    """pan/optim/muon_triton.py:127-131: p*(1-lr*wd) + u*(-lr*ratio), fp32,
    each product rounded separately."""
    wdf, neg = step_factors(lr, weight_decay, ratio)
    p = np.asarray(param, dtype=np.float32)
    u = np.asarray(update, dtype=np.float32)
    return ((p * wdf).astype(np.float32) + (u * neg).astype(np.float32)).astype(np.float32)


def _coeff_list(ns_coefficients, ns_steps):
    c = tuple(ns_coefficients)
    if len(c) == 3 and not isinstance(c[0], (tuple, list)):
        return [tuple(float(v) for v in c)] * ns_steps
    if len(c) != ns_steps:
        raise ValueError("per-iteration coefficients need one (a, b, c) per step")
    return [tuple(float(v) for v in t) for t in c]


def _ops(precision: str):
    if precision == "fp64":
        return np.float64, (lambda x: x)
    if precision == "fp32":
        return np.float32, (lambda x: np.asarray(x, dtype=np.float32))
    if precision == "bf16":
        return np.float32, round_bf16
    raise ValueError(f"unknown precision {precision!r}")


def ns_standard(G, ns_coefficients=DEFAULT_COEFFS, ns_steps: int = DEFAULT_NS_STEPS,
                eps: float = EPS, precision: str = "fp64"):
    """Standard quintic Newton–Schulz, TORCH/optim/_muon.py:31-70.

    X = G (transposed if tall), X /= max(|X|_F, eps), then per iteration
      A = X Xᵀ ; B = b A + c A A ; X = a X + B X
    and transposed back. precision:
      "fp64"  all in float64 (the exact-arithmetic reference)
      "fp32"  all in float32
      "bf16"  torch's rounding points: bf16 input (:55), bf16 norm and bf16
              divide (:59), every GEMM/addmm output rounded to bf16 (:62-66);
              products accumulate in fp32.
    """
    if ns_steps >= 100:
        raise ValueError("Number of steps must be less than 100 for computational efficiency")
    G = np.asarray(G)
    if G.ndim != 2:
        raise ValueError("Input tensor gradient must be a 2D matrix")
    dt, rnd = _ops(precision)
    coeffs = _coeff_list(ns_coefficients, ns_steps)
    X = rnd(G.astype(dt))
    tall = G.shape[0] > G.shape[1]
    if tall:
        X = np.ascontiguousarray(X.T)
    nrm = dt(math.sqrt(float(np.sum(X.astype(np.float64) ** 2))))
    if precision == "bf16":
        nrm = round_bf16(np.float32(nrm))[()]
        nrm = max(nrm, round_bf16(np.float32(eps))[()]) if not np.isnan(nrm) else nrm
    else:
        nrm = dt(max(nrm, eps)) if not np.isnan(nrm) else nrm
    X = rnd((X / nrm).astype(dt))
    for a, b, c in coeffs:
        A = rnd(X @ X.T)
        B = rnd(dt(c) * (A @ A) + dt(b) * A)
        X = rnd(dt(a) * X + B @ X)
    if tall:
        X = np.ascontiguousarray(X.T)
    return X


def ns_gram(G, ns_coefficients=DEFAULT_COEFFS, ns_steps: int = DEFAULT_NS_STEPS,
            eps: float = EPS, precision: str = "fp64"):
    """PAN 2's production NS on the Gram matrix, pan/optim/patch_muon.py:275-334.

    R = X Xᵀ; per iteration Z = c R R + b R; Q = aI + Z (first) or Q Z + a Q;
    R <- (aI+Z) R (aI+Z) via RZ = R Z + a R, R = Z RZ + a RZ; at iteration 2
    (when ns_steps > 2) X <- Q X and R is recomputed; finally X <- Q X.
    In exact arithmetic this equals ns_standard. "bf16" rounds every GEMM
    output and the diagonal add to bf16 as the bf16 quack GEMMs do.
    """
    G = np.asarray(G)
    dt, rnd = _ops(precision)
    coeffs = _coeff_list(ns_coefficients, ns_steps)
    reset = {2} if ns_steps > 2 else set()
    X = rnd(G.astype(dt))
    nrm = dt(math.sqrt(float(np.sum(X.astype(np.float64) ** 2))))
    if precision == "bf16":
        nrm = round_bf16(np.float32(nrm))[()]
    nrm = max(nrm, dt(eps))
    X = rnd((X / nrm).astype(dt))
    tall = X.shape[0] > X.shape[1]
    if tall:
        X = np.ascontiguousarray(X.T)
    M = X.shape[0]
    eye = np.eye(M, dtype=dt)
    R = rnd(X @ X.T)
    Q = None
    for i, (a, b, c) in enumerate(coeffs):
        if i in reset:
            X = rnd(Q @ X)
            R = rnd(X @ X.T)
            Q = None
        Z = rnd(dt(c) * (R @ R) + dt(b) * R)
        if Q is None:
            Q = rnd(Z + dt(a) * eye)
        else:
            Q = rnd(Q @ Z + dt(a) * Q)
        if i < ns_steps - 1 and (i + 1) not in reset:
            RZ = rnd(R @ Z + dt(a) * R)
            R = rnd(Z @ RZ + dt(a) * RZ)
    X = rnd(Q @ X)
    if tall:
        X = np.ascontiguousarray(X.T)
    return X


def quintic_power(x, ns_coefficients=DEFAULT_COEFFS, ns_steps: int = DEFAULT_NS_STEPS):
    """Scalar map of NS on one singular value: x -> p(p(...p(x))),
    p(x) = a x + b x^3 + c x^5 (the iteration acts on each singular value of
    the normalised input independently)."""
    x = np.asarray(x, dtype=np.float64)
    for a, b, c in _coeff_list(ns_coefficients, ns_steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return x


def muon_step(param, grad, buf, *, lr: float, weight_decay: float, momentum: float = 0.95,
              nesterov: bool = True, ns_coefficients=DEFAULT_COEFFS, ns_steps: int = DEFAULT_NS_STEPS,
              eps: float = EPS, adjust_lr_fn=None, shape: Sequence[int] | None = None,
              ns_precision: str = "fp32", ns_form: str = "standard"):
    """One Muon step of one matrix, pan/optim/patch_muon.py:149-171, with the
    standard NS (torch's quintic) or PAN 2's gram form (ns_form="gram",
    pan/optim/patch_muon.py:275-334): returns (new_param, new_buf, O)."""
    nb, u = momentum_nesterov(buf, grad, momentum, nesterov)
    ns = {"standard": ns_standard, "gram": ns_gram}[ns_form]
    O = ns(u, ns_coefficients, ns_steps, eps, precision=ns_precision)
    ratio = adjust_lr_ratio(adjust_lr_fn, shape if shape is not None else np.shape(param))
    if ns_precision != "fp64":
        O = round_bf16(O) if ns_precision == "bf16" else O.astype(np.float32)
    p = step_param(param, O, lr, weight_decay, ratio)
    return p, nb, O


def ns_flops(rows: int, cols: int, ns_steps: int = DEFAULT_NS_STEPS):
    """(F_ns, F_dense) of one matrix: symmetric gram + symmetric A² + dense B·X,
    and the dense-equivalent count, with M the short and N the long side."""
    M, N = min(rows, cols), max(rows, cols)
    f_ns = ns_steps * (M * (M + 1) * N + M * M * (M + 1) + 2 * M * M * N)
    f_dense = ns_steps * (4 * M * M * N + 2 * M ** 3)
    return f_ns, f_dense
