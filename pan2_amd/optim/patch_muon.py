"""PAN 2's Muon step on MI355X, installed over torch.optim.Muon by :func:`patch_muon`.

Drop-in for pan/optim/patch_muon.py. ``torch.optim.Muon.step`` calls the
module-global ``torch.optim._muon._single_tensor_muon`` once per param group
(TORCH/optim/_muon.py:172-201, :345); :func:`patch_muon` replaces it (and the
standalone ``_zeropower_via_newtonschulz``) exactly as the reference does
(pan/optim/patch_muon.py:337-339). The replacement keeps the keyword interface
and hands the whole group to libpanmuon in one call: momentum, Newton–Schulz
and the parameter step for every matrix of the group run as grouped HIP
launches on the current stream, with no host synchronisation.

Newton–Schulz is the standard quintic of torch (TORCH/optim/_muon.py:61-66),
bf16 operands with fp32 accumulation; see pan2_amd/csrc/pm_kernels.hpp.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib


def _scalar_lr(lr):
    """A 1-element tensor lr becomes 0-d (pan/optim/patch_muon.py:33-35)."""
    return lr.reshape(()) if isinstance(lr, Tensor) and lr.ndim > 0 else lr


def _require_matrix(grad: Tensor) -> None:
    """pan/optim/patch_muon.py:38-40."""
    if grad.ndim != 2:
        raise ValueError(f"Muon updates 2-D weights only, got a gradient of shape {tuple(grad.shape)}")


def _adjust_ratio(adjust_lr_fn, shape) -> float:
    """Shape factor of torch.optim._muon._adjust_lr (TORCH/optim/_muon.py:73-84):
    adjusted_lr = lr * ratio."""
    return float(torch.optim._muon._adjust_lr(1.0, adjust_lr_fn, shape))


def _is_dtensor(t) -> bool:
    try:
        from torch.distributed.tensor import DTensor
    except Exception:  # pragma: no cover - torch without distributed
        return False
    return isinstance(t, DTensor)


# libpanmuon's workspace cap in bytes; 0 = the library default (12 GiB).
WORKSPACE_LIMIT = 0

# Newton–Schulz organisation: "gram" (PAN 2's _gram_newtonschulz_local,
# pan/optim/patch_muon.py:275-334, which PAN 2's single-tensor step calls for
# every matrix, :164-168, and patch_muon installs, :339) or "standard" (torch's
# quintic, TORCH/optim/_muon.py:61-66). The default is PAN 2's.
NS_FORM = "gram"


@torch.compiler.disable
def _single_tensor_muon(
    params: list[Tensor],
    grads: list[Tensor],
    muon_momentum_bufs: list[Tensor],
    *,
    lr,
    weight_decay: float,
    momentum: float,
    nesterov: bool,
    ns_coefficients,
    ns_steps: int,
    eps: float,
    adjust_lr_fn,
    has_complex: bool,
) -> None:
    """Keyword-compatible replacement of pan/optim/patch_muon.py:43-268 (one GPU).

    ``adjust_lr_fn`` may be a ``(base_fn, chunk_dim, n_chunks)`` tuple as in
    the reference (:63-68): with chunk_dim 0 each weight is orthogonalised as
    n_chunks independent row blocks and the lr is adjusted with the chunk shape
    (:142, :165-167). Chunking along dim 1 is rejected as in the reference
    (:143-144).
    """
    lr = _scalar_lr(lr)
    if has_complex:
        raise ValueError("PAN 2's Muon step has no complex-parameter path")
    if isinstance(adjust_lr_fn, tuple):
        base_adjust_lr_fn, chunk_dim, total_chunks = adjust_lr_fn
    else:
        base_adjust_lr_fn, chunk_dim, total_chunks = adjust_lr_fn, None, None
    if chunk_dim == 1:
        raise AssertionError("Chunking along dim 1 is not currently supported (previously supported without comm overlap)")
    if not params:
        return

    p_list, g_list, b_list, ratios, counts = [], [], [], [], []
    for param, grad, buf in zip(params, grads, muon_momentum_bufs):
        _require_matrix(grad)
        assert nesterov
        if _is_dtensor(param) or _is_dtensor(grad):
            raise NotImplementedError("DTensor (FSDP-sharded) Muon params need the multi-GPU path, which this "
                                      "single-GPU build does not include")
        assert buf.shape == grad.shape, "buf and grad must have the same shape"
        assert buf.is_contiguous() and grad.is_contiguous(), "buf and grad must be contiguous"
        assert param.shape == grad.shape, "param and update must have the same shape"
        assert param.is_contiguous(), "param and update must be contiguous"
        if chunk_dim == 0:
            R, N = grad.shape
            assert R % total_chunks == 0, "# rows must be divisible by # local chunks (chunks must be same-shape)"
        if not param.is_cuda:
            raise RuntimeError("pan2_amd Muon runs on HIP device tensors only; got a CPU parameter")
        if param.numel() == 0:
            continue  # torch's step leaves an empty param and its buffer as they are
        p_list.append(param)
        g_list.append(grad)
        b_list.append(buf)
        if chunk_dim == 0:
            # row blocks param[k*rows:(k+1)*rows], addressed in place by the library
            ratios.append(_adjust_ratio(base_adjust_lr_fn, (R // total_chunks, N)))
            counts.append(total_chunks)
        else:
            ratios.append(_adjust_ratio(base_adjust_lr_fn, param.shape))
            counts.append(1)

    by_device: dict[torch.device, list[int]] = {}
    for i, p in enumerate(p_list):
        by_device.setdefault(p.device, []).append(i)
    for dev, idx in by_device.items():
        _lib.muon_step(
            [p_list[i] for i in idx], [g_list[i] for i in idx], [b_list[i] for i in idx],
            [ratios[i] for i in idx], chunks=[counts[i] for i in idx],
            lr=lr, weight_decay=weight_decay, momentum=momentum, nesterov=nesterov,
            ns_coefficients=ns_coefficients, ns_steps=ns_steps, eps=eps,
            workspace_limit=WORKSPACE_LIMIT, ns_form=NS_FORM,
        )


def newton_schulz(grad: Tensor, ns_coefficients, ns_steps: int, eps: float) -> Tensor:
    """Replacement of torch.optim._muon._zeropower_via_newtonschulz
    (TORCH/optim/_muon.py:31-70; the reference installs its gram form here,
    pan/optim/patch_muon.py:339). Returns the bf16 orthogonalised update,
    shaped like ``grad`` (``[..., M, N]`` batches are orthogonalised per matrix,
    as pan/optim/patch_muon.py:275-334 allows)."""
    if ns_steps >= 100:
        raise ValueError("Number of steps must be less than 100 for computational efficiency")
    if grad.ndim < 2:
        raise ValueError("Input tensor gradient must be a 2D matrix")
    if not grad.is_cuda:
        raise RuntimeError("pan2_amd Newton–Schulz runs on HIP device tensors only")
    x = grad if grad.dtype in (torch.float32, torch.bfloat16) else grad.float()
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    if out.numel() == 0:
        return out  # torch's NS returns an empty matrix unchanged in shape
    flat_in = x.reshape(-1, *x.shape[-2:])
    flat_out = out.view(-1, *x.shape[-2:])
    _lib.newton_schulz_into([(flat_in[i], flat_out[i]) for i in range(flat_in.shape[0])],
                            ns_coefficients=ns_coefficients, ns_steps=ns_steps, eps=eps,
                            workspace_limit=WORKSPACE_LIMIT, ns_form=NS_FORM)
    return out


def patch_muon(ns_form: str | None = None) -> None:
    """Install the HIP path into torch.optim._muon (pan/optim/patch_muon.py:337-339).

    ``ns_form`` selects the Newton–Schulz organisation for every later step:
    "gram" (the reference's production _gram_newtonschulz_local, the default)
    or "standard" (torch's quintic); None keeps the current choice
    (``NS_FORM``).
    Loads libpanmuon first, so a missing or broken build fails here, loudly.
    """
    global NS_FORM
    if ns_form is not None:
        _lib.ns_form_code(ns_form)  # validates
        NS_FORM = ns_form
    _lib.load()
    torch.optim._muon._single_tensor_muon = _single_tensor_muon
    torch.optim._muon._zeropower_via_newtonschulz = newton_schulz
