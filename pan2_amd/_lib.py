"""ctypes binding of libpanmuon.so (C ABI declared in include/panmuon.h).

Every wrapper enqueues on torch's current stream of the tensors' device and
never synchronises the host. There is no fallback: if the library is missing
or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpanmuon.so")
ABI_VERSION = 2

PM_DTYPE_F32 = 0
PM_DTYPE_BF16 = 1
PM_DTYPE_F16 = 2  # pm_adam_step only

# Newton–Schulz organisation (pm_hparams.ns_form)
PM_NS_STANDARD = 0
PM_NS_GRAM = 1
NS_FORMS = {"standard": PM_NS_STANDARD, "gram": PM_NS_GRAM}

PM_EINVAL = -1
PM_EDTYPE = -2
PM_EWORKSPACE = -3
PM_EHIP = -4
PM_EUNSUPPORTED = -5

# Every symbol the header declares (checked by tests/test_abi_exports.py).
EXPORTS = (
    "pm_abi_version",
    "pm_last_error",
    "pm_workspace_bytes",
    "pm_muon_step",
    "pm_muon_step_noalloc",
    "pm_ns_workspace_bytes",
    "pm_newton_schulz",
    "pm_momentum_nesterov",
    "pm_step_param",
    "pm_gram_workspace_bytes",
    "pm_gram",
    "pm_gemm_symmetric_workspace_bytes",
    "pm_gemm_symmetric",
    "pm_timing_enable",
    "pm_timing_read",
    "pm_adam_workspace_bytes",
    "pm_adam_step",
)

KERNEL_KINDS = ("prologue", "norm", "gram", "poly", "update", "final", "qinit", "small_core", "adam", "reduce")


class PmMatrix(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("momentum", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("param_ld", ctypes.c_int64),
        ("grad_ld", ctypes.c_int64),
        ("momentum_ld", ctypes.c_int64),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("momentum_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("adj_ratio", ctypes.c_double),
    ]


# numpy twin of PmMatrix: the row blocks of a chunked param are filled as arrays
_PM_MATRIX_NP = np.dtype({
    "names": [f for f, _ in PmMatrix._fields_],
    "formats": ["u8", "u8", "u8", "i8", "i8", "i8", "i8", "i8", "i4", "i4", "i4", "i4", "f8"],
    "offsets": [getattr(PmMatrix, f).offset for f, _ in PmMatrix._fields_],
    "itemsize": ctypes.sizeof(PmMatrix),
})


class PmNsMatrix(ctypes.Structure):
    _fields_ = [
        ("in_", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("in_ld", ctypes.c_int64),
        ("out_ld", ctypes.c_int64),
        ("in_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class PmHparams(ctypes.Structure):
    _fields_ = [
        ("momentum", ctypes.c_float),
        ("nesterov", ctypes.c_int32),
        ("ns_steps", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("weight_decay", ctypes.c_double),
        ("a", ctypes.c_float),
        ("b", ctypes.c_float),
        ("c", ctypes.c_float),
        ("ns_form", ctypes.c_int32),
        ("coeffs", ctypes.POINTER(ctypes.c_float)),
        ("workspace_limit", ctypes.c_uint64),
    ]


class PmAdamTensor(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("max_exp_avg_sq", ctypes.c_void_p),
        ("step", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("exp_avg_dtype", ctypes.c_int32),
        ("exp_avg_sq_dtype", ctypes.c_int32),
    ]


class PmAdamHparams(ctypes.Structure):
    _fields_ = [
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("amsgrad", ctypes.c_int32),
        ("maximize", ctypes.c_int32),
        ("decoupled_weight_decay", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class PmLaunchTime(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("iteration", ctypes.c_int32),
        ("n_matrices", ctypes.c_int32),
        ("flops", ctypes.c_double),
        ("bytes", ctypes.c_double),
        ("ms", ctypes.c_float),
        ("reserved", ctypes.c_float),
    ]


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libpanmuon.so once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m pan2_amd.build` (needs hipcc)")
        lib = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, sz, f32, f64 = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                       ctypes.c_size_t, ctypes.c_float, ctypes.c_double)
        pm, pns, php = ctypes.POINTER(PmMatrix), ctypes.POINTER(PmNsMatrix), ctypes.POINTER(PmHparams)
        sig = {
            "pm_abi_version": (ctypes.c_int, []),
            "pm_last_error": (ctypes.c_char_p, []),
            "pm_workspace_bytes": (sz, [pm, ctypes.c_int, php]),
            "pm_muon_step": (ctypes.c_int, [pm, ctypes.c_int, php, vp, f64, vp, sz, vp]),
            "pm_muon_step_noalloc": (ctypes.c_int, [pm, ctypes.c_int, php, vp, f64, vp]),
            "pm_ns_workspace_bytes": (sz, [pns, ctypes.c_int, php]),
            "pm_newton_schulz": (ctypes.c_int, [pns, ctypes.c_int, php, vp, sz, vp]),
            "pm_momentum_nesterov": (ctypes.c_int, [vp, i32, vp, i32, vp, i32, i64, f32, i32, vp]),
            "pm_step_param": (ctypes.c_int, [vp, i32, vp, i32, i64, vp, f64, f32, f64, vp]),
            "pm_gram_workspace_bytes": (sz, []),
            "pm_gram": (ctypes.c_int, [vp, i64, i64, vp, vp, sz, vp]),
            "pm_gemm_symmetric_workspace_bytes": (sz, []),
            "pm_gemm_symmetric": (ctypes.c_int, [vp, vp, vp, vp, i64, f32, f32, vp, sz, vp]),
            "pm_timing_enable": (ctypes.c_int, [ctypes.c_int]),
            "pm_timing_read": (ctypes.c_int, [ctypes.POINTER(PmLaunchTime), ctypes.c_int]),
            "pm_adam_workspace_bytes": (sz, [ctypes.c_int]),
            "pm_adam_step": (ctypes.c_int, [ctypes.POINTER(PmAdamTensor), ctypes.c_int, ctypes.POINTER(PmAdamHparams),
                                            vp, f64, vp, vp, vp, sz, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.pm_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libpanmuon ABI {lib.pm_abi_version()} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def last_error() -> str:
    return load().pm_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Raise the reference's exception type for a failed call."""
    if rc == 0:
        return
    msg = f"{what}: {last_error()}"
    if rc in (PM_EINVAL, PM_EDTYPE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return PM_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return PM_DTYPE_BF16
    raise TypeError(f"libpanmuon supports float32 and bfloat16 tensors, got {t.dtype}")


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ns_form_code(ns_form) -> int:
    """'standard' (torch's quintic) or 'gram' (PAN 2's gram form) -> pm_hparams.ns_form."""
    if ns_form not in NS_FORMS:
        raise ValueError(f"ns_form must be one of {sorted(NS_FORMS)}, got {ns_form!r}")
    return NS_FORMS[ns_form]


def make_hparams(*, momentum=0.95, nesterov=True, ns_coefficients=(3.4445, -4.7750, 2.0315), ns_steps=5,
                 eps=1e-7, weight_decay=0.0, workspace_limit=0, ns_form="standard"):
    """PmHparams plus the ctypes array that must outlive the call (per-step coefficients)."""
    hp = PmHparams()
    hp.ns_form = ns_form_code(ns_form)
    hp.momentum = float(momentum)
    hp.nesterov = 1 if nesterov else 0
    hp.ns_steps = int(ns_steps)
    hp.eps = float(eps)
    hp.weight_decay = float(weight_decay)
    hp.workspace_limit = int(workspace_limit)
    keep = None
    coeffs = tuple(ns_coefficients)
    if len(coeffs) == 3 and not isinstance(coeffs[0], (tuple, list)):
        hp.a, hp.b, hp.c = (float(v) for v in coeffs)
        hp.coeffs = None
    else:
        if len(coeffs) != ns_steps or any(len(t) != 3 for t in coeffs):
            raise ValueError("ns_coefficients must be (a, b, c) or one (a, b, c) per step")
        flat = [float(v) for t in coeffs for v in t]
        keep = (ctypes.c_float * len(flat))(*flat)
        hp.coeffs = ctypes.cast(keep, ctypes.POINTER(ctypes.c_float))
        hp.a, hp.b, hp.c = flat[:3]
    return hp, keep


def _ld(t: torch.Tensor) -> int:
    return t.stride(0)


def _check_matrix(t: torch.Tensor, what: str) -> None:
    if t.dim() != 2:
        raise ValueError(f"{what} must be 2-D, got shape {tuple(t.shape)}")
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be a HIP device tensor; libpanmuon has no CPU path")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        raise ValueError(f"{what} needs unit column stride and row stride >= cols")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _step_matrices(params, grads, bufs, adj_ratios, chunks):
    """The pm_matrix array of a call: entry i of the lists becomes chunks[i]
    equal row blocks (one matrix each, with adj_ratios[i]), addressed in place."""
    counts = [1] * len(params) if chunks is None else [int(c) for c in chunks]
    arr = np.zeros(sum(counts), dtype=_PM_MATRIX_NP)
    dev = params[0].device
    pos = 0
    for p, g, b, r, k in zip(params, grads, bufs, adj_ratios, counts):
        _check_matrix(p, "param")
        _check_matrix(g, "grad")
        _check_matrix(b, "momentum buffer")
        if p.shape != g.shape or p.shape != b.shape:
            raise ValueError(f"param/grad/buffer shapes differ: {tuple(p.shape)}, {tuple(g.shape)}, {tuple(b.shape)}")
        if p.device != dev or g.device != dev or b.device != dev:
            raise ValueError("all tensors of one call must be on one device")
        if k < 1 or p.shape[0] % k:
            raise ValueError(f"{p.shape[0]} rows cannot be split into {k} equal row blocks")
        rows = p.shape[0] // k
        blk = arr[pos:pos + k]
        idx = np.arange(k, dtype=np.uint64)
        for field, t in (("param", p), ("grad", g), ("momentum", b)):
            blk[field] = np.uint64(t.data_ptr()) + idx * np.uint64(rows * t.stride(0) * t.element_size())
        blk["rows"], blk["cols"] = rows, p.shape[1]
        blk["param_ld"], blk["grad_ld"], blk["momentum_ld"] = _ld(p), _ld(g), _ld(b)
        blk["param_dtype"], blk["grad_dtype"], blk["momentum_dtype"] = dtype_code(p), dtype_code(g), dtype_code(b)
        blk["adj_ratio"] = float(r)
        pos += k
    return arr


NOALLOC_SCRATCH_BYTES = 256 << 20  # PM_NOALLOC_SCRATCH_BYTES


def muon_step(params, grads, bufs, adj_ratios, *, lr, weight_decay, momentum, nesterov, ns_coefficients,
              ns_steps, eps, workspace_limit: int = 0, ns_form: str = "standard", chunks=None,
              noalloc: bool = False) -> None:
    """pm_muon_step over matching lists of 2-D device tensors (updated in place).

    lr: python float, or a 1-element float tensor on the same device (read on
    the device, no host sync). chunks: per entry, the number of equal row
    blocks orthogonalised independently (None: 1 each), addressed in place
    without building views. noalloc: call pm_muon_step_noalloc, which runs in
    the library's static scratch (NOALLOC_SCRATCH_BYTES) with no workspace
    tensor; workspace_limit does not apply.
    """
    lib = load()
    if len(params) == 0:
        return
    dev = params[0].device
    arr = _step_matrices(params, grads, bufs, adj_ratios, chunks)
    n = len(arr)
    mats = arr.ctypes.data_as(ctypes.POINTER(PmMatrix))
    hp, keep = make_hparams(momentum=momentum, nesterov=nesterov, ns_coefficients=ns_coefficients,
                            ns_steps=ns_steps, eps=eps, weight_decay=weight_decay,
                            workspace_limit=workspace_limit, ns_form=ns_form)
    lr_dev, lr_host, lr_keep = None, 0.0, None
    if isinstance(lr, torch.Tensor):
        if lr.numel() != 1:
            raise ValueError("Tensor lr must be 1-element")
        if lr.device.type == "cpu":
            lr_host = float(lr.item())
        else:
            if lr.device != dev:
                raise ValueError("lr tensor must be on the params' device")
            lr_keep = lr.reshape(()).to(torch.float32)
            lr_dev = lr_keep.data_ptr()
    else:
        lr_host = float(lr)
    with torch.cuda.device(dev):
        if noalloc:
            rc = lib.pm_muon_step_noalloc(mats, n, ctypes.byref(hp), lr_dev, lr_host, stream_of(dev))
            check(rc, "pm_muon_step_noalloc")
            del keep, lr_keep, arr
            return
        nbytes = lib.pm_workspace_bytes(mats, n, ctypes.byref(hp))
        if nbytes == 0:
            check(PM_EINVAL, "pm_workspace_bytes")
        ws = workspace(nbytes, dev)
        rc = lib.pm_muon_step(mats, n, ctypes.byref(hp), lr_dev, lr_host, ws.data_ptr(), nbytes, stream_of(dev))
    check(rc, "pm_muon_step")
    del keep, lr_keep, arr


def newton_schulz_into(pairs, *, ns_coefficients=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7,
                       workspace_limit: int = 0, ns_form: str = "standard") -> None:
    """pm_newton_schulz over [(input, output)] pairs; outputs are bf16, same shape."""
    lib = load()
    n = len(pairs)
    if n == 0:
        return
    dev = pairs[0][0].device
    mats = (PmNsMatrix * n)()
    for i, (x, o) in enumerate(pairs):
        _check_matrix(x, "input")
        _check_matrix(o, "output")
        if o.dtype != torch.bfloat16 or o.shape != x.shape:
            raise ValueError("output must be bf16 and shaped like the input")
        m = mats[i]
        m.in_, m.out = x.data_ptr(), o.data_ptr()
        m.rows, m.cols = x.shape
        m.in_ld, m.out_ld = _ld(x), _ld(o)
        m.in_dtype = dtype_code(x)
    hp, keep = make_hparams(ns_coefficients=ns_coefficients, ns_steps=ns_steps, eps=eps,
                            workspace_limit=workspace_limit, ns_form=ns_form)
    with torch.cuda.device(dev):
        nbytes = lib.pm_ns_workspace_bytes(mats, n, ctypes.byref(hp))
        if nbytes == 0:
            check(PM_EINVAL, "pm_ns_workspace_bytes")
        ws = workspace(nbytes, dev)
        rc = lib.pm_newton_schulz(mats, n, ctypes.byref(hp), ws.data_ptr(), nbytes, stream_of(dev))
    check(rc, "pm_newton_schulz")
    del keep


def momentum_nesterov_into(buf, grad, update, momentum: float, nesterov: bool = True) -> None:
    lib = load()
    for t, w in ((buf, "buf"), (grad, "grad"), (update, "update")):
        if not t.is_cuda:
            raise RuntimeError(f"{w} must be a HIP device tensor")
        if not t.is_contiguous():
            raise AssertionError(f"{w} must be contiguous")
    if buf.shape != grad.shape or update.shape != grad.shape:
        raise AssertionError("buf, grad and update must have the same shape")
    with torch.cuda.device(buf.device):
        rc = lib.pm_momentum_nesterov(buf.data_ptr(), dtype_code(buf), grad.data_ptr(), dtype_code(grad),
                                      update.data_ptr(), dtype_code(update), buf.numel(), float(momentum),
                                      1 if nesterov else 0, stream_of(buf.device))
    check(rc, "pm_momentum_nesterov")


def step_param_inplace(param, update, lr, weight_decay: float, adj_ratio: float) -> None:
    lib = load()
    for t, w in ((param, "param"), (update, "update")):
        if not t.is_cuda:
            raise RuntimeError(f"{w} must be a HIP device tensor")
        if not t.is_contiguous():
            raise AssertionError(f"{w} must be contiguous")
    if param.shape != update.shape:
        raise AssertionError("param and update must have the same shape")
    lr_dev, lr_host, keep = None, 0.0, None
    if isinstance(lr, torch.Tensor):
        if lr.device.type == "cpu":
            lr_host = float(lr.item())
        else:
            keep = lr.reshape(()).to(torch.float32)
            lr_dev = keep.data_ptr()
    else:
        lr_host = float(lr)
    with torch.cuda.device(param.device):
        rc = lib.pm_step_param(param.data_ptr(), dtype_code(param), update.data_ptr(), dtype_code(update),
                               param.numel(), lr_dev, lr_host, float(weight_decay), float(adj_ratio),
                               stream_of(param.device))
    check(rc, "pm_step_param")
    del keep


def gram(x: torch.Tensor) -> torch.Tensor:
    """Symmetric X Xᵀ in bf16 through pm_gram (rows and cols multiples of 256)."""
    lib = load()
    _check_matrix(x, "x")
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("pm_gram takes a contiguous bf16 matrix")
    rows, cols = x.shape
    out = torch.empty((rows, rows), dtype=torch.bfloat16, device=x.device)
    with torch.cuda.device(x.device):
        nbytes = lib.pm_gram_workspace_bytes()
        ws = workspace(nbytes, x.device)
        rc = lib.pm_gram(x.data_ptr(), rows, cols, out.data_ptr(), ws.data_ptr(), nbytes, stream_of(x.device))
    check(rc, "pm_gram")
    return out


def gemm_symmetric(left: torch.Tensor, right: torch.Tensor, addend: torch.Tensor | None = None, *,
                   alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """alpha * left @ right.T + beta * addend through pm_gemm_symmetric (bf16, m x m,
    m a multiple of 256; the upper triangle is computed and mirrored)."""
    lib = load()
    mats = [(left, "left"), (right, "right")] + ([(addend, "addend")] if addend is not None else [])
    m = left.shape[0]
    for t, w in mats:
        _check_matrix(t, w)
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != (m, m):
            raise ValueError(f"{w} must be a contiguous bf16 {m}x{m} matrix")
    if beta != 0.0 and addend is None:
        raise ValueError("beta != 0 needs an addend")
    out = torch.empty((m, m), dtype=torch.bfloat16, device=left.device)
    with torch.cuda.device(left.device):
        nbytes = lib.pm_gemm_symmetric_workspace_bytes()
        ws = workspace(nbytes, left.device)
        rc = lib.pm_gemm_symmetric(left.data_ptr(), right.data_ptr(),
                                   addend.data_ptr() if addend is not None else None, out.data_ptr(), m,
                                   float(alpha), float(beta), ws.data_ptr(), nbytes, stream_of(left.device))
    check(rc, "pm_gemm_symmetric")
    return out


def _device_scalar(t, what: str, dev):
    """Pointer of a 1-element float32 device tensor (or None)."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or t.numel() != 1 or t.dtype != torch.float32 or t.device != dev:
        raise ValueError(f"{what} must be a 1-element float32 tensor on {dev}")
    return t.data_ptr()


# numpy twin of PmAdamTensor (the array _pm_host.fill_adam writes)
_PM_ADAM_NP = np.dtype({
    "names": [f for f, _ in PmAdamTensor._fields_],
    "formats": ["u8", "u8", "u8", "u8", "u8", "u8", "i8", "i4", "i4", "i4", "i4"],
    "offsets": [getattr(PmAdamTensor, f).offset for f, _ in PmAdamTensor._fields_],
    "itemsize": ctypes.sizeof(PmAdamTensor),
})


ADAM_DTYPES = {torch.float32: PM_DTYPE_F32, torch.bfloat16: PM_DTYPE_BF16, torch.float16: PM_DTYPE_F16}

_host = None


def host_ext():
    """The _pm_host extension (pan2_amd/csrc/pm_host.cpp, built beside libpanmuon
    by pan2_amd.build): fills pm_adam_tensor arrays from torch's tensor lists."""
    global _host
    if _host is None:
        try:
            from . import _pm_host
        except ImportError as e:
            raise RuntimeError("pan2_amd._pm_host is not built; run `python -m pan2_amd.build`") from e
        if _pm_host.DESC_BYTES != ctypes.sizeof(PmAdamTensor):
            raise RuntimeError(f"_pm_host's pm_adam_tensor is {_pm_host.DESC_BYTES} bytes, "
                               f"ctypes' {ctypes.sizeof(PmAdamTensor)}: rebuild")
        _host = _pm_host
    return _host


def adam_dtype_code(t: torch.Tensor) -> int:
    """pm_adam_step's dtype code of a tensor: float32, bfloat16 or float16."""
    code = ADAM_DTYPES.get(t.dtype)
    if code is None:
        raise TypeError(f"pm_adam_step supports float32, bfloat16 and float16 tensors, got {t.dtype}")
    return code


def adam_descs(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps):
    """The pm_adam_tensor array of one call, filled in one C++ pass, or None
    when some tensor is off params[0]'s HIP device, of a dtype pm_adam_step
    does not take (float32 / bfloat16 / float16; max_exp_avg_sq of
    exp_avg_sq's dtype; float32 steps), not contiguous, or of another element
    count than its param. max_exp_avg_sqs: [] without amsgrad."""
    h = host_ext()
    arr = np.empty(len(params), dtype=_PM_ADAM_NP)
    rc = h.fill_adam(arr.ctypes.data, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps)
    return arr if rc == h.FILLED else None


def _check_adam_lists(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, amsgrad, dev):
    for i, p in enumerate(params):
        x = max_exp_avg_sqs[i] if amsgrad else None
        named = ((grads[i], "grad"), (exp_avgs[i], "exp_avg"), (exp_avg_sqs[i], "exp_avg_sq"))
        for t, what in ((p, "param"),) + named + (((x, "max_exp_avg_sq"),) if amsgrad else ()):
            if t.device != dev:
                raise ValueError("all tensors of one call must be on one device")
            if not t.is_contiguous():
                raise ValueError(f"{what} must be contiguous")
            if t.shape != p.shape:
                raise ValueError(f"{what} shape {tuple(t.shape)} differs from the param's {tuple(p.shape)}")
            adam_dtype_code(t)
        st = state_steps[i]
        if st.device != dev or st.dtype != torch.float32 or st.numel() != 1:
            raise ValueError("state steps must be 1-element float32 tensors on the params' device")
        if amsgrad and x.dtype != exp_avg_sqs[i].dtype:
            raise ValueError("max_exp_avg_sq must have exp_avg_sq's dtype")


def adam_step(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, *, lr, beta1: float,
              beta2: float, eps: float, weight_decay: float, amsgrad: bool, maximize: bool, decoupled: bool,
              grad_scale=None, found_inf=None, trusted: bool = False) -> None:
    """pm_adam_step over matching lists of contiguous device tensors (updated
    in place, steps included). lr: float, or a 1-element tensor (read on the
    device when it lives there). max_exp_avg_sqs: read with amsgrad only.
    trusted: the lists come from torch's Adam, whose _init_group already
    guarantees one device, matching shapes and float32 device steps; the
    descriptor pass still checks devices, dtypes, element counts and
    contiguity."""
    n = len(params)
    if n == 0:
        return
    dev = params[0].device
    if not params[0].is_cuda:
        raise RuntimeError("pan2_amd Adam runs on HIP device tensors only; got a CPU parameter")
    if not trusted:
        _check_adam_lists(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, amsgrad, dev)
    arr = adam_descs(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs if amsgrad else [], state_steps)
    if arr is None:
        raise ValueError("pm_adam_step takes contiguous float32 / bfloat16 / float16 tensors of their param's "
                         "size on one HIP device, max_exp_avg_sq of exp_avg_sq's dtype and float32 steps")
    adam_launch(arr, dev, lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
                maximize=maximize, decoupled=decoupled, grad_scale=grad_scale, found_inf=found_inf)


def adam_launch(arr, dev, *, lr, beta1: float, beta2: float, eps: float, weight_decay: float, amsgrad: bool,
                maximize: bool, decoupled: bool, grad_scale=None, found_inf=None) -> None:
    """pm_adam_step over a filled pm_adam_tensor array (adam_descs) of tensors
    on device dev, on its current stream."""
    lib = load()
    n = len(arr)
    keep = [arr]
    hp = PmAdamHparams(beta1=float(beta1), beta2=float(beta2), eps=float(eps), weight_decay=float(weight_decay),
                       amsgrad=int(bool(amsgrad)), maximize=int(bool(maximize)),
                       decoupled_weight_decay=int(bool(decoupled)))
    lr_dev, lr_host = None, 0.0
    if isinstance(lr, torch.Tensor):
        if lr.numel() != 1:
            raise ValueError("Tensor lr must be 1-element")
        if lr.device.type == "cpu":
            lr_host = float(lr.item())
        else:
            if lr.device != dev:
                raise ValueError("lr tensor must be on the params' device")
            lr_t = lr.reshape(()).to(torch.float32)
            keep.append(lr_t)
            lr_dev = lr_t.data_ptr()
    else:
        lr_host = float(lr)
    gs = _device_scalar(grad_scale, "grad_scale", dev)
    fi = _device_scalar(found_inf, "found_inf", dev)
    with torch.cuda.device(dev):
        nbytes = lib.pm_adam_workspace_bytes(n)
        ws = workspace(nbytes, dev)
        rc = lib.pm_adam_step(arr.ctypes.data_as(ctypes.POINTER(PmAdamTensor)), n, ctypes.byref(hp), lr_dev,
                              lr_host, gs, fi, ws.data_ptr(), nbytes, stream_of(dev))
    check(rc, "pm_adam_step")
    del keep


def timing_enable(on: bool = True) -> None:
    """Record a HIP event after every library launch (bench instrumentation)."""
    load().pm_timing_enable(1 if on else 0)


def timing_read(max_records: int = 1 << 16) -> list[dict]:
    """Wait for the recorded launches and return one dict per launch."""
    lib = load()
    buf = (PmLaunchTime * max_records)()
    n = lib.pm_timing_read(buf, max_records)
    if n < 0:
        check(n, "pm_timing_read")
    return [dict(kind=KERNEL_KINDS[r.kind], group=r.group, iteration=r.iteration, n_matrices=r.n_matrices,
                 flops=r.flops, bytes=r.bytes, ms=r.ms) for r in buf[:n]]
