"""Benchmark: one full Muon step (momentum + Newton–Schulz + param step) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 5]

A step is one ``torch.optim.Muon.step()`` through the drop-in API
(pan2_amd.optim.patch_muon installed, tensor lr on the device) over a
BASELINE config's synthetic parameter set, already resident in HBM. Prints one
JSON line. ``value`` is the NS TFLOP/s of the whole step (F_ns / step time);
``roofline`` is the Newton–Schulz GEMM kernel alone, from HIP events recorded
by libpanmuon on the launch stream over the timed steps; ``cpu_baseline`` is
the reference's CPU path (stock torch Muon, float lr) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

S = 5120
BLOCK = ([(S, S)] * 8 + [(4 * S, S)] * 2 + [(S, 4 * S)] * 2 + [(S, 6 * S)] * 2 + [(4096, S)])
CONFIGS = {
    1: ("single_1024x4096_fp32", [(1024, 4096)]),
    2: ("attn_proj_48x5120sq", [(S, S)] * 48),
    3: ("mlp_16up_16down", [(4 * S, S)] * 16 + [(S, 4 * S)] * 16),
    4: ("mmdit_block_ragged", BLOCK),
    5: ("mmdit_24_blocks", BLOCK * 24),
    # not a BASELINE config: PAN 2's chunked QKV weights, 44 joint blocks of
    # (2 x 3 x 4096, 4096), each orthogonalised as 192 row blocks of 128 x 4096
    # (pan/models/transformers/pan_transformer.py:65-71, pan/optim/patch_muon.py:75-142)
    6: ("qkv_chunks_44x192", [(6 * 4096, 4096)] * 44),
}
CHUNKS = {6: 192}  # row blocks per param (adjust_lr_fn = (base, 0, n))

# Not a BASELINE config: the AdamW half of PAN 2's step. The params Muon leaves
# to AdamW (pan/optim/muon.py:12-92) in the 29B MMDiT (hidden 4096, 44 joint
# blocks): per block the qkv / out / FFN biases, the q/k norm weights and the
# text modulation vector (pan/models/transformers/pan_transformer.py:66-68,
# :148, :205-212, :297), plus the embedders and the head (:732, :801; the
# timestep MLP, patch embedding and output head shapes are approximations).
H = 4096
ADAMW_BLOCK = [(6 * H,), (2 * H,), (8 * H,), (H,), (4 * H,), (H,), (256,), (256,), (6 * H,)]
ADAMW_GLOBAL = [(3, H), (H,), (H, H), (H,), (H, 256), (H,), (H, H), (H,), (H, 64), (H,), (64, H), (64,),
                (2 * H, H), (2 * H,)]
ADAMW_SET = ADAMW_BLOCK * 44 + ADAMW_GLOBAL
CONFIGS[7] = ("adamw_pan2_set", [])


def unit_shapes(config: int):
    """The matrices Newton–Schulz runs on: the params, or their row blocks."""
    n = CHUNKS.get(config, 1)
    return [(r // n, c) for r, c in CONFIGS[config][1] for _ in range(n)]


def ns_flops(shape, steps=5):
    m, n = min(shape), max(shape)
    return steps * (m * (m + 1) * n + m * m * (m + 1) + 2 * m * m * n)


def dense_flops(shape, steps=5):
    m, n = min(shape), max(shape)
    return steps * (4 * m * m * n + 2 * m ** 3)


def gram_form_flops(shape, steps=5):
    """Algorithmic FLOPs of PAN 2's gram form (pan/optim/patch_muon.py:275-334):
    two symmetric grams, two applications Q X, and the symmetric M^3 products
    (Z every iteration, Q from the second of a segment, RZ and R unless the
    next iteration resets or ends)."""
    m, n = min(shape), max(shape)
    reset = 2 if steps > 2 else -1
    sym, segment_start = 0, True
    for i in range(steps):
        if i == reset:
            segment_start = True
        sym += 1 if segment_start else 2
        segment_start = False
        if i + 1 < steps and i + 1 != reset:
            sym += 2
    grams = 2 if reset >= 0 else 1
    applies = 2 if reset >= 0 else 1
    return grams * m * (m + 1) * n + sym * m * m * (m + 1) + applies * 2 * m * m * n


def build_state(shapes, config, device, seed=1234):
    """Params/grads/momentum resident on the device (BASELINE dtypes)."""
    import torch

    fp32 = config == 1
    pdt = torch.float32 if fp32 else torch.bfloat16
    gen = torch.Generator(device=device).manual_seed(seed)
    params, moms = [], []
    for shape in shapes:
        p = torch.nn.Parameter(torch.empty(shape, dtype=pdt, device=device))
        p.data.normal_(0.0, 0.02, generator=gen)
        p.grad = torch.empty(shape, dtype=pdt, device=device)
        p.grad.normal_(0.0, 1.0 if fp32 else 1e-3, generator=gen)
        m = torch.empty(shape, dtype=torch.float32, device=device)
        if fp32:
            m.zero_()
        else:
            m.normal_(0.0, 1e-3, generator=gen)
        params.append(p)
        moms.append(m)
    return params, moms


GEMM_KERNEL = "pm_ns_gemm_kernel"
COPY_KERNEL = "__amd_rocclr_copyBuffer"
# kernels whose HBM traffic per launch bench.py reports: the name in the
# profiler's CSV (a prefix of the demangled name) and the summary file's stem
TRAFFIC_KERNELS = {
    "gemm": ("pm_ns_gemm_kernel", "pm_ns_gemm_kernel"),
    "small_update": ("pm_small_apply_kernel<2, 1, ", "pm_small_apply_kernel_update"),
}


def traffic_path(workload: str, kernel: str = "gemm") -> str:
    return os.path.join(ROOT, "profiles", f"{TRAFFIC_KERNELS[kernel][1]}_{workload}_traffic.json")


def traffic_bytes(workload: str, kernel: str = "gemm", ns_form: str = "standard"):
    """HBM bytes per launch of the kernel from the committed counter summary,
    or None. The summaries are measured on the standard form (the default
    bench command), so a gram-form line reports None."""
    path = traffic_path(workload, kernel)
    if ns_form != "standard" or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["bytes_per_launch"]


def _counter_by_dispatch(path: str, counter: str) -> dict:
    import csv

    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Dispatch_Id"], r["Kernel_Name"])
            out[key] = out.get(key, 0.0) + float(r["Counter_Value"])
    return out


def traffic_summary(args) -> int:
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the launches of
    --traffic-kernel (the GEMM engine by default), each scaled by what the same
    counter reads for the calibration copy (copy_mib MiB read and written).
    Writes the JSON that bench.py reports as traffic."""
    kname = TRAFFIC_KERNELS[args.traffic_kernel][0]
    if not (args.fetch_csv and args.write_csv and args.copy_mib):
        print("--traffic-summary needs --fetch-csv, --write-csv and --copy-mib", file=sys.stderr)
        return 2
    known_kib = args.copy_mib * 1024.0
    result = {}
    for counter, path in (("FETCH_SIZE", args.fetch_csv), ("WRITE_SIZE", args.write_csv)):
        vals = _counter_by_dispatch(path, counter)
        # the calibration copies are the last three copy dispatches of the run
        # (the counter may read a fixed fraction of the bytes: that fraction is
        # the scale)
        copies = [v for (d, k), v in sorted(vals.items(), key=lambda kv: int(kv[0][0])) if COPY_KERNEL in k][-3:]
        gemm = [v for (d, k), v in vals.items() if kname in k]
        if not copies or not gemm:
            print(f"{counter}: no calibration copy or no {kname} dispatches in {path}", file=sys.stderr)
            return 1
        copy_kib = sum(copies) / len(copies)
        scale = known_kib / copy_kib
        result[counter] = {"copy_kib": copy_kib, "scale": scale, "gemm_launches": len(gemm),
                           "gemm_kib_mean_raw": sum(gemm) / len(gemm),
                           "gemm_bytes_mean": sum(gemm) / len(gemm) * scale * 1024.0}
    out = {"kernel": kname, "copy_mib": args.copy_mib,
           "bytes_per_launch": result["FETCH_SIZE"]["gemm_bytes_mean"] + result["WRITE_SIZE"]["gemm_bytes_mean"],
           "fetch": result["FETCH_SIZE"], "write": result["WRITE_SIZE"]}
    with open(args.traffic_summary, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))
    return 0


def hbm_stream(device, mib: int = 2048, reps: int = 5) -> dict:
    """What plain streams reach on this box's HBM, beside the 8 TB/s peak the
    HBM rooflines are quoted against: torch's device copy (mib MiB read + mib
    written) and a fill (mib MiB written), best of reps, by HIP events on the
    current stream. Run after the timed region."""
    import torch

    n = (mib << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]

    def best(fn):
        fn()
        ms = []
        for _ in range(reps):
            ev[0].record()
            fn()
            ev[1].record()
            ev[1].synchronize()
            ms.append(ev[0].elapsed_time(ev[1]))
        return min(ms)

    nbytes = n * 4
    out = {
        "copy_gbs": round(2 * nbytes / (best(lambda: dst.copy_(src)) * 1e-3) / 1e9, 1),
        "write_gbs": round(nbytes / (best(lambda: dst.fill_(2.0)) * 1e-3) / 1e9, 1),
        "mib": mib,
    }
    del src, dst
    return out


def bench_adamw(args) -> int:
    """One AdamW.step() over PAN 2's AdamW param set (fp32 params, grads and
    state, tensor lr): libpanmuon's pm_adam_step behind torch's fused AdamW,
    timed beside torch's own fused AdamW (the reference's GPU path) on the
    same box."""
    import math

    import torch

    import pan2_amd.optim.patch_adamw as pa
    from pan2_amd import _lib

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stock = pa._adam_module._fused_adam
    steps = max(args.steps, 20)
    warmup = max(args.warmup, 3)
    gen = torch.Generator(device=device).manual_seed(7)
    numel = sum(math.prod(s) for s in ADAMW_SET)
    bytes_per_step = 28.0 * numel  # param r+w, grad r, exp_avg r+w, exp_avg_sq r+w (fp32)

    def build():
        ps = []
        for shape in ADAMW_SET:
            p = torch.nn.Parameter(torch.empty(shape, device=device))
            p.data.normal_(0.0, 0.02, generator=gen)
            p.grad = torch.empty(shape, device=device).normal_(0.0, 1e-3, generator=gen)
            ps.append(p)
        return torch.optim.AdamW(ps, lr=torch.tensor(1e-4, device=device), betas=(0.95, 0.95), eps=1e-8,
                                 weight_decay=0.05, fused=True)

    def timed(opt, fn):
        pa._adam_module._fused_adam = fn
        for _ in range(warmup):
            opt.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            opt.step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    print(f"bench: AdamW set, {len(ADAMW_SET)} tensors, {numel} params", file=sys.stderr, flush=True)
    try:
        ref_ms = timed(build(), stock)
        ours = build()
        _lib.load()
        pa._adam_module._fused_adam = pa._fused_adam
        for _ in range(warmup):
            ours.step()
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        _lib.timing_read()
        t0 = time.perf_counter()
        for _ in range(steps):
            ours.step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        recs = [r for r in _lib.timing_read() if r["kind"] == "adam"]
        _lib.timing_enable(False)
    finally:
        pa._adam_module._fused_adam = stock
    kern_ms = sum(r["ms"] for r in recs) / max(1, len(recs))
    achieved = bytes_per_step / (kern_ms * 1e-3) / 1e9 if kern_ms > 0 else 0.0
    stream = hbm_stream(device)
    cpu = None
    if not args.no_cpu_baseline:
        # torch's CPU AdamW (foreach) over the same set, one timed step after one warmup
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        cps = []
        g = torch.Generator().manual_seed(7)
        for shape in ADAMW_SET:
            p = torch.nn.Parameter(torch.randn(shape, generator=g) * 0.02)
            p.grad = torch.randn(shape, generator=g) * 1e-3
            cps.append(p)
        copt = torch.optim.AdamW(cps, lr=1e-4, betas=(0.95, 0.95), eps=1e-8, weight_decay=0.05, foreach=True)
        copt.step()
        t0 = time.perf_counter()
        copt.step()
        cms = (time.perf_counter() - t0) * 1e3
        cpu = {"value": round(bytes_per_step / (cms * 1e-3) / 1e9, 2), "unit": "GB/s", "step_ms": round(cms, 2),
               "cores": threads, "kind": "reference",
               "sample": "torch.optim.AdamW(foreach=True) step on the host over the whole fp32 set (one step after "
                         "a warmup step)"}
    out = {
        "metric": "AdamW step GB/s (algorithmic HBM bytes / step time), 1 GPU",
        "value": round(bytes_per_step / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "adamw_pan2_set", "baseline_config": None, "tensors": len(ADAMW_SET),
                   "params": numel, "param_dtype": "fp32", "grad_dtype": "fp32", "state_dtype": "fp32",
                   "bytes_per_step": bytes_per_step},
        "reference_gpu": {"what": "torch's own fused AdamW (torch._fused_adamw_) on the same box",
                          "ms_per_step": round(ref_ms, 4),
                          "value": round(bytes_per_step / (ref_ms * 1e-3) / 1e9, 2), "unit": "GB/s"},
        "roofline": {"kernel": "pm_adam_kernel", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": None, "avg_launch_ms": round(kern_ms, 4)},
        "hbm_stream": stream,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", type=int, default=5, choices=sorted(CONFIGS))
    ap.add_argument("--ns-form", default="standard", choices=("standard", "gram"),
                    help="standard: torch's quintic (the BASELINE metric); gram: PAN 2's production gram form, "
                         "reported with its own (smaller) executed FLOP count")
    ap.add_argument("--no-gram-form", action="store_true",
                    help="skip the second measurement: the same config stepped with the gram form (PAN 2's "
                         "production Newton-Schulz, the drop-in's default) after the standard-form timing")
    ap.add_argument("--cpu-budget", type=float, default=45.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-gpu", action="store_true",
                    help="skip the stock torch.optim.Muon step on the GPU (reference_gpu)")
    ap.add_argument("--workspace-gib", type=float, default=0.0, help="libpanmuon workspace cap (0 = default)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after timing, run a plain device copy of this many MiB 3x (HBM counter calibration)")
    ap.add_argument("--traffic-summary", metavar="OUT_JSON",
                    help="offline: turn rocprofv3 FETCH_SIZE / WRITE_SIZE CSVs of a --copy-mib run into HBM bytes "
                         "per GEMM launch (needs --fetch-csv, --write-csv, --copy-mib)")
    ap.add_argument("--fetch-csv")
    ap.add_argument("--write-csv")
    ap.add_argument("--traffic-kernel", default="gemm", choices=sorted(TRAFFIC_KERNELS),
                    help="--traffic-summary: whose launches (gemm: the NS GEMM engine; small_update: the small-matrix "
                         "UPDATE apply)")
    args = ap.parse_args()
    if args.traffic_summary:
        return traffic_summary(args)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design, not code", file=sys.stderr)
        return 2
    if args.config == 7:
        return bench_adamw(args)

    import torch
    import torch.optim._muon as torch_muon

    # torch's stock Muon functions, kept for the CPU baseline before patching
    stock_fns = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
    import pan2_amd.optim.patch_muon as pm
    from pan2_amd import _lib
    from pan2_amd.optim.patch_muon import patch_muon

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    name, shapes = CONFIGS[args.config]
    print(f"bench: config {args.config} ({name}), {len(shapes)} matrices, building state", file=sys.stderr, flush=True)
    t0 = time.time()
    params, moms = build_state(shapes, args.config, device)
    patch_muon(ns_form=args.ns_form)
    if args.workspace_gib:
        pm.WORKSPACE_LIMIT = int(args.workspace_gib * (1 << 30))
    lr = torch.tensor(0.02, dtype=torch.float32, device=device)
    group = {"params": params}
    if args.config in CHUNKS:
        group["adjust_lr_fn"] = ("match_rms_adamw", 0, CHUNKS[args.config])
    opt = torch.optim.Muon([group], lr=lr, weight_decay=0.01, momentum=0.95, adjust_lr_fn="match_rms_adamw")
    for p, m in zip(params, moms):
        opt.state[p]["momentum_buffer"] = m
    torch.cuda.synchronize()
    print(f"bench: state ready in {time.time() - t0:.1f}s; warmup {args.warmup}", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    print("bench: warmup done; timing", file=sys.stderr, flush=True)

    _lib.timing_enable(True)
    _lib.timing_read()  # clear
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    host = 0.0  # time inside step() calls: host work, as the GPU work is enqueued without waiting
    for _ in range(args.steps):
        h0 = time.perf_counter()
        opt.step()
        host += time.perf_counter() - h0
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    recs = _lib.timing_read()
    _lib.timing_enable(False)
    # (not in counter runs: its copies would join the calibration copies)
    stream = None if args.copy_mib else hbm_stream(device)
    if args.copy_mib:
        # HBM counter calibration: a copy kernel that reads and writes exactly copy_mib MiB
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    ms_per_step = elapsed * 1e3 / args.steps
    print(f"bench: {ms_per_step:.2f} ms/step", file=sys.stderr, flush=True)

    units = unit_shapes(args.config)
    f_ns = sum(ns_flops(s) for s in units)
    f_dense = sum(dense_flops(s) for s in units)
    # the gram form does less work than the quintic: its rate is its own executed FLOPs over time
    f_run = f_ns if args.ns_form == "standard" else sum(gram_form_flops(s) for s in units)
    value = f_run / (ms_per_step * 1e-3) / 1e12

    # the GEMM engine's launches, K-split reduces included (their epilogues are the stage's)
    gemm = [r for r in recs if r["kind"] in ("gram", "poly", "update", "final", "reduce")]
    gemm_ms = sum(r["ms"] for r in gemm)
    gemm_flops = sum(r["flops"] for r in gemm)
    achieved = gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0
    if args.config in CHUNKS:
        # row blocks of at most 128 rows run on the small-matrix kernels, which
        # are HBM-bound: the roofline is the dominant one, the apply of
        # X <- a·X + S·X, at 4 algorithmic bytes per element (X read once, X'
        # written once)
        ups = [r for r in recs if r["kind"] == "update"]
        um, un = units[0]
        up_ms = sum(r["ms"] for r in ups)
        up_bytes = sum(4.0 * um * un * r["n_matrices"] for r in ups)
        gbs = up_bytes / (up_ms * 1e-3) / 1e9 if up_ms > 0 else 0.0
        roofline = {"kernel": "pm_small_apply_kernel<UPDATE>", "bound": "hbm", "achieved": round(gbs, 1),
                    "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                    "traffic": traffic_bytes(name, "small_update", args.ns_form), "bytes_per_element": 4, "launches": len(ups),
                    "avg_launch_ms": round(up_ms / max(1, len(ups)), 3)}
    else:
        roofline = {
            "kernel": "pm_ns_gemm_kernel",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic_bytes(name, ns_form=args.ns_form),
            "launches": len(gemm),
            "avg_launch_ms": round(gemm_ms / max(1, len(gemm)), 3),
        }
    stages = {}
    for kind in ("prologue", "norm", "gram", "poly", "qinit", "small_core", "update", "final", "reduce"):
        rs = [r for r in recs if r["kind"] == kind]
        if not rs:
            continue
        ms = sum(r["ms"] for r in rs) / args.steps
        entry = {"ms_per_step": round(ms, 3), "launches_per_step": len(rs) // args.steps}
        fl = sum(r["flops"] for r in rs)
        by = sum(r["bytes"] for r in rs)
        if fl:
            entry["tflops"] = round(fl / (sum(r["ms"] for r in rs) * 1e-3) / 1e12, 1)
        if by:
            entry["gbs"] = round(by / (sum(r["ms"] for r in rs) * 1e-3) / 1e9, 1)
        stages[kind] = entry

    # The reference's production organisation (gram form) on the same state,
    # after the headline timing: its own executed FLOPs over its step time.
    gram_form = None
    if args.ns_form == "standard" and not args.no_gram_form and not args.copy_mib:
        patch_muon(ns_form="gram")
        for _ in range(max(1, args.warmup)):
            opt.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            opt.step()
        torch.cuda.synchronize()
        g_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        f_gf = sum(gram_form_flops(s) for s in units)
        gram_form = {"ms_per_step": round(g_ms, 3), "f_gram_form": f_gf,
                     "executed_tflops": round(f_gf / (g_ms * 1e-3) / 1e12, 1),
                     "pct_peak_executed": round(100 * f_gf / (g_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                     "steps": args.steps}
        print(f"bench: gram form {g_ms:.2f} ms/step", file=sys.stderr, flush=True)
        patch_muon(ns_form=args.ns_form)

    # The reference's own PyTorch path on the same GPU and state, after the
    # headline timing: stock torch.optim.Muon (torch's
    # _zeropower_via_newtonschulz, one param at a time on hipBLASLt's bf16
    # GEMMs, TORCH/optim/_muon.py:31-70) with a float lr, as the reference runs
    # it without its patch (pan/optim/muon.py:126-128). Its momentum buffers
    # are torch's own, zeros_like(grad) (torch's lerp takes no fp32 buffer with
    # bf16 grads). Not for chunked groups, whose tuple adjust_lr_fn only the
    # patched step takes.
    ref_gpu = None
    if not args.no_torch_gpu and not args.copy_mib and args.config not in CHUNKS:
        ours = (torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon)
        torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = stock_fns
        torch.cuda.empty_cache()
        try:
            ref_opt = torch.optim.Muon([{"params": params}], lr=0.02, weight_decay=0.01, momentum=0.95,
                                       adjust_lr_fn="match_rms_adamw")
            ref_opt.step()
            torch.cuda.synchronize()
            r_steps = min(args.steps, 2)
            t0 = time.perf_counter()
            for _ in range(r_steps):
                ref_opt.step()
            torch.cuda.synchronize()
            r_ms = (time.perf_counter() - t0) * 1e3 / r_steps
        finally:
            torch_muon._zeropower_via_newtonschulz, torch_muon._single_tensor_muon = ours
        del ref_opt
        torch.cuda.empty_cache()
        ref_gpu = {"what": "stock torch.optim.Muon step on the same GPU, params and grads (torch's "
                           "_zeropower_via_newtonschulz, one param at a time, hipBLASLt bf16 GEMMs, float lr, "
                           "torch's own momentum buffers)",
                   "ms_per_step": round(r_ms, 3), "value": round(f_ns / (r_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                   "steps": r_steps, "speedup": round(r_ms / ms_per_step, 3)}
        print(f"bench: stock torch Muon on the GPU {r_ms:.2f} ms/step", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        from oracle.cpu_baseline import baseline

        print("bench: CPU baseline (stock torch Muon, host cores)", file=sys.stderr, flush=True)
        cb = baseline(units, budget_s=args.cpu_budget, stock_fns=stock_fns)
        cpu = {
            "value": round(f_ns / (cb["step_ms"] * 1e-3) / 1e12, 4),
            "unit": "TFLOP/s",
            "step_ms": round(cb["step_ms"], 1),
            "cores": cb["cores"],
            "kind": "reference",
            "sample": ("stock torch.optim.Muon step (the reference's float-lr path, pan/optim/muon.py:126-154), "
                       f"fp32, one matrix per distinct shape ({', '.join(cb['timed_shapes'])}) timed on "
                       f"{cb['cores']} host threads (one warm-up step, then the median of {cb['repeats']} "
                       "steps per shape); " + ("extrapolated to the config's counts by shape"
                                               if cb["extrapolated"] else "full config")),
            "cpu": cb["cpu"],
        }

    params_total = sum(s[0] * s[1] for s in shapes)
    out = {
        "metric": "Newton–Schulz TFLOP/s (% MI355X bf16 MFMA peak); Muon step ms, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": name,
            "baseline_config": args.config if args.config <= 5 else None,
            "matrices": len(units),
            "params": params_total,
            "param_dtype": "fp32" if args.config == 1 else "bf16",
            "grad_dtype": "fp32" if args.config == 1 else "bf16",
            "momentum_dtype": "fp32",
            "ns_steps": 5,
            "ns_form": args.ns_form,
            "f_ns": f_ns,
            "f_dense": f_dense,
            **({"f_gram_form": f_run} if args.ns_form == "gram" else {}),
        },
        "pct_peak_step": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "host_ms_per_step": round(host * 1e3 / args.steps, 3),
        "roofline": roofline,
        "hbm_stream": stream,
        "stages": stages,
        "gram_form": gram_form,
        "reference_gpu": ref_gpu,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
