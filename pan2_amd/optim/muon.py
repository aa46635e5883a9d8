"""Muon/AdamW parameter split and optimizer factory (drop-in for pan/optim/muon.py).

Same names, arguments, return value and errors as the reference factory
(pan/optim/muon.py:12-178). The only difference is what a tensor lr installs:
:func:`pan2_amd.optim.patch_muon.patch_muon` and
:func:`pan2_amd.optim.patch_adamw.patch_adamw`, whose steps run on libpanmuon.
"""
from __future__ import annotations

from collections import defaultdict
from typing import Dict, List, Tuple

import torch

from .patch_adamw import patch_adamw
from .patch_lr_scheduler import patch_lr_scheduler
from .patch_muon import patch_muon

# Name rules that keep a 2-D weight on AdamW (pan/optim/muon.py:24-50). The
# lists must match the reference's so the same parameters land in Muon.
_ADAMW_SUBSTRINGS = (
    "embedding", "embed_tokens", "token_embed", "token_emb", "pos_embed", "position_embed",
    "lm_head", "output_head", "classifier",
)
_ADAMW_MODULATION = (".modulation.", "text_modulation")
_ADAMW_PREFIXES = ("output_head.", "timestep_encoder.", "text_type_embedding", "patch_embed.")


def _looks_like_embedding_or_head(name: str) -> bool:
    """True for embeddings, output heads, modulation/gating layers and the PAN
    transformer's conditioning stacks (pan/optim/muon.py:12-52)."""
    key = name.lower()
    return (any(s in key for s in _ADAMW_SUBSTRINGS)
            or any(s in key for s in _ADAMW_MODULATION)
            or key.startswith(_ADAMW_PREFIXES))


_STAT_KEYS = (
    "trainable_param_tensors", "muon_param_tensors", "adamw_param_tensors",
    "muon_param_numel", "adamw_param_numel", "excluded_embedding_or_head_tensors",
)


def split_params_for_native_muon(
    model,
) -> Tuple[List[Tuple[str, torch.nn.Parameter]], List[Tuple[str, torch.nn.Parameter]], Dict[str, int]]:
    """(muon named params, adamw named params, stats), pan/optim/muon.py:55-92.

    A trainable parameter goes to Muon iff it is 2-D and its name is not an
    embedding/head/modulation name; everything else goes to AdamW.
    """
    muon, adamw = [], []
    stats = dict.fromkeys(_STAT_KEYS, 0)
    for name, p in model.named_parameters():
        if not p.requires_grad:
            continue
        stats["trainable_param_tensors"] += 1
        excluded = _looks_like_embedding_or_head(name)
        if p.ndim == 2 and not excluded:
            muon.append((name, p))
            stats["muon_param_tensors"] += 1
            stats["muon_param_numel"] += p.numel()
            continue
        adamw.append((name, p))
        stats["adamw_param_tensors"] += 1
        stats["adamw_param_numel"] += p.numel()
        if p.ndim == 2 and excluded:
            stats["excluded_embedding_or_head_tensors"] += 1
    return muon, adamw, stats


def build_native_muon_optimizers(
    model,
    *,
    lr=1e-3,
    momentum=0.95,
    weight_decay=0.1,
    muon_adjust_lr_fn="match_rms_adamw",
    adamw_betas=(0.95, 0.95),
    adamw_eps=1e-8,
    capturable=False,
    muon_chunks: dict[str, tuple[int, int]] | None = None,
):
    """Build torch.optim.Muon + fused AdamW (pan/optim/muon.py:95-178).

    Returns {"optimizers": {"muon": ..., "adamw": ...} (absent keys omitted),
    "stats": split summary, "param_names": {"muon", "adamw", "muon_chunked"}}.
    A tensor ``lr`` installs the libpanmuon steps (Muon, and the fused AdamW
    behind the AdamW half) and the host-side get_last_lr; a float lr leaves
    torch's stock Muon in place, as the reference does (:126-128). ``muon_chunks`` maps a param name to
    (chunk_dim, n_chunks); each distinct pair becomes its own param group whose
    ``adjust_lr_fn`` is (muon_adjust_lr_fn, dim, n_chunks) (:130-146).
    """
    if not hasattr(torch.optim, "Muon"):
        raise RuntimeError(
            "torch.optim.Muon is not available in this PyTorch build. "
            f"Installed torch version: {torch.__version__}. Please upgrade to a version that includes torch.optim.Muon."
        )
    muon_named, adamw_named, stats = split_params_for_native_muon(model)
    chunks = muon_chunks or {}
    tensor_lr = isinstance(lr, torch.Tensor)

    def _lr():
        return lr.clone() if tensor_lr else lr

    optimizers: Dict[str, torch.optim.Optimizer] = {}
    if muon_named:
        if tensor_lr:
            patch_muon()
            patch_lr_scheduler()
        regular = [p for name, p in muon_named if name not in chunks]
        by_chunk: dict[tuple[int, int], list] = defaultdict(list)
        for name, p in muon_named:
            if name in chunks:
                by_chunk[chunks[name]].append(p)
        groups: list[dict] = [{"params": regular}]
        groups += [{"params": ps, "adjust_lr_fn": (muon_adjust_lr_fn, dim, n)}
                   for (dim, n), ps in by_chunk.items()]
        optimizers["muon"] = torch.optim.Muon(
            groups, lr=_lr(), weight_decay=weight_decay, momentum=momentum, adjust_lr_fn=muon_adjust_lr_fn,
        )
    if adamw_named:
        if tensor_lr:
            patch_adamw()
        optimizers["adamw"] = torch.optim.AdamW(
            adamw_named, lr=_lr(), betas=adamw_betas, eps=adamw_eps, weight_decay=weight_decay,
            capturable=capturable, fused=True,
        )
    if not optimizers:
        raise ValueError("No trainable parameters found to build optimizers.")
    return {
        "optimizers": optimizers,
        "stats": stats,
        "param_names": {
            "muon": [n for n, _ in muon_named if n not in chunks],
            "adamw": [n for n, _ in adamw_named],
            "muon_chunked": [(n, *chunks[n]) for n, _ in muon_named if n in chunks],
        },
    }
