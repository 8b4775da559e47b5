#!/usr/bin/env python3
"""Benchmark of the gfx950 attention forward on its BASELINE.json metric.

One step = one attention forward over the north-star workload
(B=1, H=16, Sq=Skv=16384, D=128, fp16, scale 1/sqrt(D)), inputs already
resident in HBM. Prints one JSON line with the driver's fields plus:

* ``roofline``: the kernel's algorithmic TFLOP/s (4*B*H*Sq*Skv*D per launch,
  flops_probe.py:18) from the average launch duration measured with HIP events
  on the stream the kernel runs on, against MI355X's dense fp16 MFMA peak;
  ``traffic`` is the HBM bytes per launch read from the committed rocprofv3
  counter summary (profiles/), or null when that file is absent.
* ``launches``: minimum and median single-launch duration over up to 20
  further launches after the timed region, each between its own event pair.
* ``counters``: MFMA busy % and LDS bank-conflict % from the committed
  rocprofv3 summary, with the workload they were measured on, and
  ``driver_form``: the committed per-dispatch reconciliation of this command's
  short form (SQ clock x useful MFMA cycles against the measured frac).
* ``cpu_baseline``: torch SDPA MATH on the host CPU (the oracle's routine)
  over the whole workload, chunked by head and 2048 query rows (with
  ``--workload c1`` .. ``c5`` that config's, c5 on its first 256 query rows of
  every head against all keys).
* ``configs``: kernel rates of BASELINE.json's configs c2-c5, each timed the
  same way after the north star's timed region (not part of it).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-configs]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn fwd TFLOP/s + % fp16 MFMA peak, B1 H16 S16K D128, 1×MI355X"
PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
PEAK_HBM_TBS = 8.0  # MI355X HBM3E
WORKLOAD = dict(B=1, H=16, Sq=16384, Skv=16384, D=128)
SEED = 106
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_fwd_ns_pmc.txt")
# Cycles x clock against frac for the north star under the driver's command.
DRIVER_FORM_FILE = os.path.join(ROOT, "profiles", "attn_fwd_ns_driver_form.txt")
DRIVER_FORM_KEYS = ("driver_form_sq_clock_ghz", "driver_form_mfma_busy_pct",
                    "driver_form_useful_mfma_pct", "driver_form_predicted_frac",
                    "driver_form_measured_frac")
CONV_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "conv3d_vae_kernel_trace.txt")
WARMUP_MS = 250.0  # default warm-up: about this much back-to-back work ...
MIN_WARMUP = 30  # ... and at least this many launches
MAX_WARMUP = 20000
# The reference's D = 512 benchmark (bench_d512.py:21, :63): one VAE mid-block
# head, B1 H1 D512, q, k, v ~ N(0,1), at these sequence lengths.
VAE_D512 = {"vae1k": 1024, "vae4k": 4096, "vae9k": 9216, "vae129k": 129600}


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The card climbs from about 1.5 to 1.87 GHz over the first tens of
    # milliseconds of sustained matrix load, then holds. Without --warmup,
    # the untimed launches run for about WARMUP_MS of back-to-back work (at
    # least MIN_WARMUP launches), so the 50 timed launches measure the steady
    # state a model's layers run in whatever the kernel's length; an explicit
    # --warmup W runs exactly W.
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip timing the other BASELINE configs after the north star")
    ap.add_argument("--torch-sdpa", action="store_true",
                    help="also time torch's fused scaled_dot_product_attention (flash backend, "
                         "else memory-efficient) on the same inputs, the same way")
    ap.add_argument("--workload", default="ns",
                    choices=["ns", "ns_h8", "c1", "c2", "c3", "c4", "c5", *VAE_D512,
                             "conv3d_vae"],
                    help="BASELINE.json config to run (default: the north star the metric is "
                         "quoted on; others are for profiling: ns_h8 is the north star with 8 "
                         "of its 16 heads, the same kernel and per-workgroup work at half the "
                         "cycles, for counters that would saturate on the full workload; "
                         "vae1k .. vae129k are the reference's D = 512 benchmark shapes, one "
                         "head of 1024 to 129600 tokens; conv3d_vae times the conv3d kernel on "
                         "a 512->512 3x3x3 VAE layer)")
    ap.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"],
                    help="attention input type (profiling; the metric is quoted for fp16)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="instead of attention, time a plain device copy of this many bytes "
                         "(reference point for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def warm_up(call, requested):
    """Runs the untimed launches and returns how many ran: exactly
    ``requested`` when given, else enough for about WARMUP_MS of back-to-back
    launches (sized by the host time of one synchronised launch, which
    over-counts short kernels' length and so errs towards fewer), at least
    MIN_WARMUP and at most MAX_WARMUP."""
    import torch

    if requested is not None:
        for _ in range(requested):
            call()
        torch.cuda.synchronize()
        return requested
    call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    call()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-6)
    n = min(MAX_WARMUP, max(MIN_WARMUP, math.ceil(WARMUP_MS * 1e-3 / one)))
    for _ in range(n - 2):
        call()
    torch.cuda.synchronize()
    return n


def copy_calibration(nbytes, steps):
    """Plain HBM copy of `nbytes` per launch: its FETCH_SIZE / WRITE_SIZE per
    dispatch, divided by nbytes, is the scale factor for the counter runs."""
    import torch

    x = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    x.random_(0, 255)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        y.copy_(x)
    b.record()
    b.synchronize()
    ms = a.elapsed_time(b) / steps
    print(json.dumps({"copy_bytes": nbytes, "ms": round(ms, 4),
                      "GB_per_s_read_plus_write": round(2 * nbytes / ms / 1e6, 1)}), flush=True)


def read_profile_figures(path=TRAFFIC_FILE):
    """HBM bytes per launch, counter ratios and the workload the counters were
    measured on, from a committed summary's "name: value" lines."""
    out = {"traffic": None, "mfma_busy_pct": None, "lds_bank_conflict_pct": None,
           "counters_workload": None}
    if not os.path.isfile(path):
        return out
    with open(path) as f:
        text = f.read()
    for key, name in (("traffic", "hbm_bytes_per_launch"), ("mfma_busy_pct", "mfma_busy_pct"),
                      ("lds_bank_conflict_pct", "lds_bank_conflict_pct")):
        m = re.search(rf"^{name}\s*[:=]\s*([0-9.eE+-]+)", text, re.M)
        if m:
            out[key] = float(m.group(1))
    m = re.search(r"^counters_workload\s*[:=]\s*(.+)$", text, re.M)
    if m:
        out["counters_workload"] = m.group(1).strip()
    return out


def read_driver_form_figures(path=DRIVER_FORM_FILE):
    """The committed driver-form reconciliation (per-dispatch SQ clock and
    MFMA-busy cycles against the measured frac), or None without the file."""
    if not os.path.isfile(path):
        return None
    with open(path) as f:
        text = f.read()
    out = {}
    for name in DRIVER_FORM_KEYS:
        m = re.search(rf"^{name}\s*[:=]\s*([0-9.eE+-]+)", text, re.M)
        out[name[len("driver_form_"):]] = float(m.group(1)) if m else None
    out["note"] = ("a profiling session of `bench.py --steps 20 --warmup 5`, not this run: "
                   "useful = busy x 32/34 (2 of 34 MFMAs per block carry row sums); "
                   "predicted frac = useful x clock / 2.4 GHz")
    out["source"] = os.path.relpath(path, ROOT)
    return out


def conv3d_cpu_baseline(x, w, b):
    """The oracle's implicit GEMM (numpy fp64, oracle/conv3d.py) on the host CPU
    over one of the layer's six output depth slices (min of 2)."""
    import numpy as np

    from oracle.conv3d import conv3d_gemm

    xs = x[:, :, 0:3].float().cpu().numpy().astype(np.float16)  # -> one output slice
    wn, bn = w.float().cpu().numpy().astype(np.float16), b.float().cpu().numpy().astype(np.float16)
    ts = []
    for _ in range(2):
        t0 = time.perf_counter()
        conv3d_gemm(xs, wn, bn)
        ts.append(time.perf_counter() - t0)
    t = min(ts)
    try:  # BLAS threads numpy used
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 0) for i in threadpool_info()
                       if i.get("user_api") == "blas"), default=0) or os.cpu_count()
    except Exception:  # noqa: BLE001 - threadpoolctl missing or failing
        threads = os.cpu_count()
    k, c, kt, kr, ks = wn.shape
    m = xs.shape[0] * (xs.shape[2] - kt + 1) * (xs.shape[3] - kr + 1) * (xs.shape[4] - ks + 1)
    flops = 2 * m * k * c * kt * kr * ks
    return {
        "value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
        "kind": "port",
        "sample": (f"oracle conv3d_gemm (numpy im2col + fp64 GEMM on {threads} BLAS threads) on "
                   f"output depth slice 1 of 6 ({m} voxels), min of 2: {t:.3f} s; "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def conv3d_bench(args):
    """conv3d kernel on a VAE decoder layer: x [1, 512, 8, 64, 64] NDHWC fp16,
    w [512, 512, 3, 3, 3], bias; one JSON line (profiling, not the metric)."""
    import torch

    import gfx906_amd
    from gfx906_amd import kitchen

    g = torch.Generator().manual_seed(7)
    n, c, d, h, wd, k, t = 1, 512, 8, 64, 64, 512, 3
    cl = torch.channels_last_3d
    x = (torch.randn(n, c, d, h, wd, generator=g) * 0.25).half().cuda().contiguous(memory_format=cl)
    w = (torch.randn(k, c, t, t, t, generator=g) * 0.25).half().cuda().contiguous(memory_format=cl)
    b = torch.randn(k, generator=g).half().cuda()
    z, p, q = d - t + 1, h - t + 1, wd - t + 1
    out = torch.empty(n, k, z, p, q, dtype=torch.float16, device="cuda").contiguous(
        memory_format=cl)
    dims = [n, d, h, wd, c, k, t, t, t, 1, 1, 1, z, p, q]
    xs, os_ = list(kitchen.packed_strides(x.shape)), list(kitchen.packed_strides(out.shape))
    conv = gfx906_amd.extension().conv3d

    def call():
        conv(x, w, b, None, out, dims, xs, os_, [0, 0, 0, 0])

    warmup = warm_up(call, args.warmup)
    avg, wall = time_region(call, args.steps)
    flops = 2 * n * z * p * q * k * c * t ** 3
    achieved = flops / (avg * 1e-3) / 1e12
    print(json.dumps({
        "metric": "conv3d fwd TFLOP/s (fp16 NDHWC implicit GEMM), 1xMI355X",
        "value": round(flops * args.steps / wall / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4), "higher_is_better": True,
        "dtype": "fp16", "data": "synthetic: x, w ~ 0.25 N(0,1), bias ~ N(0,1), seeded",
        "config": {"workload": "conv3d x[1,512,8,64,64] w[512,512,3,3,3] stride 1, bias"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS, 4),
                     "traffic": read_profile_figures(CONV_TRAFFIC_FILE)["traffic"],
                     "kernel_ms_avg": round(avg, 4),
                     "algorithmic_flops_per_launch": flops},
        "cpu_baseline": None if args.no_cpu else conv3d_cpu_baseline(x, w, b)}), flush=True)


def cpu_baseline(w=WORKLOAD, mults=(1.0, 1.0), seed=SEED, rows=None):
    """torch SDPA MATH on the host CPU (fp32 upcast of the same fp16 inputs,
    the oracle's routine) over the whole workload: every head and query row,
    chunked per head and by 2048 query rows (chunk times summed); one warm-up
    chunk, then the best of 2 full passes. `rows`: only the first `rows` query
    rows of every head, against the full key range (c5's seeded 256-row slice,
    BASELINE.json)."""
    import torch

    from oracle.attention import chunked_sdpa_math, make_inputs

    q, k, v = make_inputs(w["B"], w["H"], w["Sq"], w["Skv"], w["D"], *mults, seed=seed)
    if rows is not None:
        q = q[:, :, :rows]
    scale = w["D"] ** -0.5
    chunked_sdpa_math(q[:, :1, :2048], k[:, :1], v[:, :1], scale)  # warm-up
    best = float("inf")
    for _ in range(2):
        t0 = time.perf_counter()
        chunked_sdpa_math(q, k, v, scale)
        best = min(best, time.perf_counter() - t0)
    flops = 4 * q.shape[0] * q.shape[1] * q.shape[2] * w["Skv"] * w["D"]
    what = ("the whole workload" if rows is None else
            f"the first {rows} query rows of every head against all {w['Skv']} keys")
    return {
        "value": round(flops / best / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"torch SDPA MATH (fp32 upcast) on CPU over {what}: B={w['B']}, "
                   f"{w['H']} heads, Sq={w['Sq']}, Skv={w['Skv']}, D={w['D']}, chunked by "
                   f"2048 query rows (times summed), best of 2 passes after a warm-up chunk: "
                   f"{best:.3f} s; os.cpu_count()={os.cpu_count()}"),
    }


def torch_sdpa_leg(attn, q, k, v, scale, flops, args):
    """torch.nn.functional.scaled_dot_product_attention with its flash backend
    (else the memory-efficient one; never the math path) on the same contiguous
    inputs, timed like the kernel: warm-up, then args.steps launches between
    HIP events on the current stream. None when neither backend serves the call."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    sdpa = torch.nn.functional.scaled_dot_product_attention
    ours = attn(q, k, v, scale)
    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel(backend):
                ref = sdpa(q, k, v, scale=scale)
                torch.cuda.synchronize()
                warm_up(lambda: sdpa(q, k, v, scale=scale), args.warmup)
                avg, _ = time_region(lambda: sdpa(q, k, v, scale=scale), args.steps)
        except RuntimeError:  # backend cannot serve this shape or dtype
            continue
        achieved = flops / (avg * 1e-3) / 1e12
        return {"backend": backend.name, "kernel_ms_avg": round(avg, 4),
                "achieved": round(achieved, 2), "frac": round(achieved / PEAK_TFLOPS, 4),
                "max_abs_vs_kernel": (ref.float() - ours.float()).abs().max().item()}
    return None


def time_region(call, steps):
    """`steps` back-to-back launches between two HIP events on the current
    stream (the stream the kernels run on), bracketed by synchronisations.
    Returns (average ms per launch from the events, wall-clock seconds of the
    same region on the host). One event pair over the region, not one per
    launch: an event between launches adds its own few microseconds to short
    kernels."""
    import torch

    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        call()
    b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return a.elapsed_time(b) / steps, wall


def launch_spread(call, n):
    """Minimum and median duration (ms) of single launches: `n` further
    launches after the timed region, each between its own pair of HIP events
    on the current stream. Reported beside the timed region's average, never
    in its place (the events between launches add their own few microseconds
    to short kernels)."""
    import torch

    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda.synchronize()
    for a, b in evs:
        a.record(stream)
        call()
        b.record(stream)
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    return {"n": n, "ms_min": round(ms[0], 4), "ms_median": round(ms[n // 2], 4),
            "pass": "single launches, one HIP event pair each, after the timed region"}


CONFIG_LEGS = ("c2", "c3", "c4", "c5")


def other_configs(attn, steps):
    """Kernel rates of BASELINE.json configs c2-c5, measured in this run after
    the north star's timed region (outside it): seeded fp16 inputs (the
    oracle's generator, as the parity tests use), then for each config about
    WARMUP_MS of untimed launches (the card lowers its clock while the inputs
    are generated on the host) and `steps` launches timed with HIP events."""
    import gfx906_amd
    from oracle.attention import CONFIGS, make_inputs

    out = {}
    for name in CONFIG_LEGS:
        B, H, Sq, Skv, D, qm, vm, seed = CONFIGS[name]
        q, k, v = (t.to("cuda") for t in make_inputs(B, H, Sq, Skv, D, qm, vm, seed=seed))
        scale = D ** -0.5
        flops = gfx906_amd.flops(B, H, Sq, Skv, D)
        warmup = warm_up(lambda: attn(q, k, v, scale), None)
        avg, _ = time_region(lambda: attn(q, k, v, scale), steps)
        achieved = flops / (avg * 1e-3) / 1e12
        out[name] = {"shape": f"B{B} H{H} Sq{Sq} Skv{Skv} D{D}", "kernel_ms_avg": round(avg, 4),
                     "achieved": round(achieved, 2), "frac": round(achieved / PEAK_TFLOPS, 4),
                     "warmup": warmup, "steps": steps}
        del q, k, v
    out["measured"] = ("in this run, after the north star's timed region; TFLOP/s from the "
                       "average launch time (HIP events over the timed launches), "
                       "4*B*H*Sq*Skv*D FLOP per launch")
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the attention shards over heads with no communication)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.copy_bytes:
        copy_calibration(args.copy_bytes, args.steps)
        return

    if args.workload == "conv3d_vae":
        conv3d_bench(args)
        return

    import gfx906_amd
    from oracle.attention import CONFIGS, make_inputs

    if args.workload == "ns":
        w, mults, seed = WORKLOAD, (1.0, 1.0), SEED
    elif args.workload == "ns_h8":
        w, mults, seed = dict(WORKLOAD, H=8), (1.0, 1.0), SEED
    elif args.workload in VAE_D512:
        S = VAE_D512[args.workload]
        w, mults, seed = dict(B=1, H=1, Sq=S, Skv=S, D=512), (1.0, 1.0), SEED
    else:
        B, H, Sq, Skv, D, qm, vm, seed = CONFIGS[args.workload]
        w, mults = dict(B=B, H=H, Sq=Sq, Skv=Skv, D=D), (qm, vm)
    dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    q, k, v = (t.to("cuda", dt) for t in make_inputs(w["B"], w["H"], w["Sq"], w["Skv"], w["D"],
                                                      *mults, seed=seed))
    scale = w["D"] ** -0.5
    attn = gfx906_amd.extension().attn
    flops = gfx906_amd.flops(w["B"], w["H"], w["Sq"], w["Skv"], w["D"])

    warmup = warm_up(lambda: attn(q, k, v, scale), args.warmup)

    # HIP events on the stream the kernel runs on (the current stream) over
    # the timed launches, and the host clock over the same region.
    avg_ms, wall = time_region(lambda: attn(q, k, v, scale), args.steps)
    ms_per_step = wall * 1e3 / args.steps
    value = flops * args.steps / wall / 1e12
    achieved = flops / (avg_ms * 1e-3) / 1e12
    spread = launch_spread(lambda: attn(q, k, v, scale), min(args.steps, 20))
    min_bytes = 2 * (2 * w["B"] * w["H"] * w["Sq"] * w["D"]
                     + 2 * w["B"] * w["H"] * w["Skv"] * w["D"])

    # The committed counter summary covers the north-star fp16 kernel only.
    north_star = args.workload == "ns" and args.dtype == "fp16"
    prof = (read_profile_figures() if north_star else
            {"traffic": None, "mfma_busy_pct": None, "lds_bank_conflict_pct": None,
             "counters_workload": None})
    metric = METRIC if args.workload == "ns" else (
        f"attn fwd TFLOP/s + % fp16 MFMA peak, config {args.workload} "
        f"(B{w['B']} H{w['H']} Sq{w['Sq']} Skv{w['Skv']} D{w['D']}), 1×MI355X")
    result = {
        "metric": metric,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": f"synthetic: q,k,v ~ N(0,1) {args.dtype} from a seeded CPU generator",
        "config": {"workload": (f"attn_fwd B{w['B']} H{w['H']} Sq{w['Sq']} Skv{w['Skv']} "
                                f"D{w['D']} {args.dtype}, scale 1/sqrt(D), no mask ("
                                + ("BASELINE.json north star" if args.workload == "ns"
                                   else "the reference's bench_d512.py shape"
                                   if args.workload in VAE_D512
                                   else f"BASELINE.json config {args.workload}") + ")"), **w,
                   "parallelism": "single GPU"},
        "pct_peak": round(100 * value / PEAK_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS, 4),
            "traffic": prof["traffic"],
            "kernel_ms_avg": round(avg_ms, 4),
            "algorithmic_flops_per_launch": flops,
            "min_hbm_bytes_per_launch": min_bytes,
            # the same minimum bytes over the launch time against 8 TB/s, and
            # the softmax's exponentials per launch (one per query-key pair)
            "min_hbm_frac": round(min_bytes / (avg_ms * 1e-3) / (PEAK_HBM_TBS * 1e12), 4),
            "exp_per_launch": w["B"] * w["H"] * w["Sq"] * w["Skv"],
        },
        "launches": spread,
        "counters": {"mfma_busy_pct": prof["mfma_busy_pct"],
                     "lds_bank_conflict_pct": prof["lds_bank_conflict_pct"],
                     "workload": prof["counters_workload"],
                     "source": os.path.relpath(TRAFFIC_FILE, ROOT)
                     if north_star and os.path.isfile(TRAFFIC_FILE) else None,
                     "driver_form": read_driver_form_figures() if north_star else None},
    }
    if args.torch_sdpa:
        result["torch_sdpa"] = torch_sdpa_leg(attn, q, k, v, scale, flops, args)
    if args.workload == "ns" and args.dtype == "fp16" and not args.no_configs:
        del q, k, v
        result["configs"] = other_configs(attn, args.steps)
    if not args.no_cpu and args.workload == "ns" and args.dtype == "fp16":
        result["cpu_baseline"] = cpu_baseline()
    elif not args.no_cpu and args.workload in CONFIGS and args.dtype == "fp16":
        result["cpu_baseline"] = cpu_baseline(w, mults, seed,
                                              rows=256 if args.workload == "c5" else None)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
