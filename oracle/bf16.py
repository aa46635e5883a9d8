"""bf16 rounding in numpy (test infrastructure; see oracle/__init__.py).

bf16 keeps the top 16 bits of an IEEE fp32. Conversion rounds to nearest,
ties to even, as torch's ``Tensor.bfloat16()`` does (torch/optim/_muon.py:55
casts the NS input this way) and as gfx950's v_cvt_pk_bf16_f32 does.
"""
import numpy as np


def round_bf16(x) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32 (exact)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = (u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)
    # NaN: keep sign and payload top bits, force quiet
    r = np.where(np.isnan(x), (u >> np.uint64(16)) | np.uint64(0x40), r)
    out = (r.astype(np.uint32) & np.uint32(0xFFFF)) << np.uint32(16)
    return out.view(np.float32).reshape(x.shape)


def to_bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of round_bf16(x)."""
    return (round_bf16(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """fp32 values of uint16 bf16 bit patterns."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)
