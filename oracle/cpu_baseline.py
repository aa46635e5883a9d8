"""CPU baseline: the reference's own CPU path, timed on the host (test infrastructure).

With a float lr the reference factory leaves torch's stock Muon unpatched
(pan/optim/muon.py:126-128) and builds it with momentum 0.95, Nesterov, the
default quintic coefficients, 5 NS steps and adjust_lr_fn="match_rms_adamw"
(pan/optim/muon.py:148-154). That stock path (TORCH/optim/_muon.py:285-318)
runs on host cores through ATen/oneDNN; this module times one ``step()`` of
it per distinct matrix shape, on fp32 params/grads/momentum (the reference's
training dtypes, train.py:573-575), and extrapolates to a config's counts.
Only bench.py's CPU-baseline leg uses it.
"""
from __future__ import annotations

import os
import platform
import statistics
import time
from collections import Counter

import torch


def cpu_info() -> dict:
    model = platform.processor() or ""
    flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                if line.startswith("flags"):
                    flags = line
                    break
    except OSError:
        pass
    return {"model": model, "avx512_bf16": "avx512_bf16" in flags, "amx_bf16": "amx_bf16" in flags}


def time_stock_muon_step(shape, *, threads: int, seed: int = 0, repeats=1, warmup: bool = False,
                         adjust_lr_fn="match_rms_adamw", stock_fns=None) -> float:
    """Seconds for one stock torch.optim.Muon step on one fp32 matrix (median).

    repeats: a count, or a function of the warm-up step's seconds giving the
    count (then the warm-up runs whatever `warmup` says).
    stock_fns: (zeropower, single_tensor_muon) to install while timing, for
    processes where patch_muon already replaced torch's module globals.
    """
    import torch.optim._muon as tm

    torch.set_num_threads(threads)
    g = torch.Generator("cpu").manual_seed(seed)
    p = torch.nn.Parameter(torch.randn(*shape, generator=g) * 0.02)
    p.grad = torch.randn(*shape, generator=g) * 1e-3
    opt = torch.optim.Muon([p], lr=0.02, weight_decay=0.01, momentum=0.95, adjust_lr_fn=adjust_lr_fn)
    saved = (tm._zeropower_via_newtonschulz, tm._single_tensor_muon)
    if stock_fns is not None:
        tm._zeropower_via_newtonschulz, tm._single_tensor_muon = stock_fns
    try:
        if warmup or callable(repeats):
            t0 = time.perf_counter()
            opt.step()
            if callable(repeats):
                repeats = repeats(time.perf_counter() - t0)
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            opt.step()
            times.append(time.perf_counter() - t0)
    finally:
        tm._zeropower_via_newtonschulz, tm._single_tensor_muon = saved
    return statistics.median(times)


def baseline(shapes, *, threads: int | None = None, budget_s: float = 45.0, stock_fns=None) -> dict:
    """Time one matrix per distinct shape and extrapolate to the full list.

    Every shape timed gets one warm-up step, then the median of 3 steps (5 for
    a step under 2% of the budget). Shapes are taken smallest first; once the
    budget is spent, the shapes not yet timed are scaled from the largest timed
    one by dense NS work (and the result is labelled extrapolated).

    Returns {"step_ms": extrapolated ms for all shapes, "cores": threads,
    "sample": description, "per_shape_ms": {...}}.
    """
    if threads is None:
        threads = len(os.sched_getaffinity(0))
    counts = Counter(tuple(s) for s in shapes)
    per_shape = {}
    spent = 0.0
    repeats_used = {}
    for shape in sorted(counts, key=lambda s: s[0] * s[1]):
        if spent > budget_s:
            break
        t0 = time.perf_counter()

        def reps(first, shape=shape):  # from the warm-up step's time
            repeats_used[shape] = 5 if first < 0.02 * budget_s else 3
            return repeats_used[shape]

        per_shape[shape] = time_stock_muon_step(shape, threads=threads, stock_fns=stock_fns, repeats=reps)
        spent += time.perf_counter() - t0
    missing = [s for s in counts if s not in per_shape]
    if missing:
        # scale the largest timed shape by dense NS work for shapes not timed
        ref = max(per_shape, key=lambda s: s[0] * s[1])

        def work(s):
            m, n = min(s), max(s)
            return 4 * m * m * n + 2 * m ** 3

        for s in missing:
            per_shape[s] = per_shape[ref] * work(s) / work(ref)
    total = sum(per_shape[s] * c for s, c in counts.items())
    timed = [s for s in per_shape if s not in missing]
    return {
        "step_ms": total * 1e3,
        "cores": threads,
        "torch_threads": torch.get_num_threads(),
        "per_shape_ms": {f"{s[0]}x{s[1]}": per_shape[s] * 1e3 for s in per_shape},
        "timed_shapes": [f"{s[0]}x{s[1]}" for s in timed],
        "repeats": {f"{s[0]}x{s[1]}": repeats_used[s] for s in timed},
        "extrapolated": len(shapes) > len(timed),
        "cpu": cpu_info(),
    }
