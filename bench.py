#!/usr/bin/env python
"""Headline benchmark of dcnv2_amd on one MI355X.

Metric: DCNv2 forward TFLOPS by the reference README formula
(README.md:17-19: B*Hout*Wout*Cout*(10*kh*kw*C + 2*kh*kw)) at the README shape
B8 C64 128x128 Cout256 3x3 fp16, plus forward+backward
milliseconds at the same shape (config 2).

A step is one forward over one batch of synthetic inputs already resident in
HBM.  The warm-up runs W untimed steps and keeps going until at least
--settle-ms of forward work has run (the GPU reaches its steady shader clock
only after some tens of milliseconds of load; the count actually run is
reported as ``warmup_steps_run``), then K steps are timed, bracketed by device
synchronisation and HIP events on the stream the kernels run on.

The ``roofline`` object covers the dominant kernel (the fused forward
kernel): achieved = algorithmic GEMM FLOPs per launch (2*B*Cout*Hout*Wout*C*
kh*kw) / its average duration, measured with the library's per-stage HIP
events (recorded on the launch stream) over a second timed loop.  The other
configurations (c2 forward+backward, c3, c4) are reported beside it with the
same per-stage timing and fractions.  ``cpu_baseline`` times the float32 CPU
oracle (oracle/dcn_oracle.c, OpenMP) on bounded samples of c0, c1 and c2.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]

Profiling aids (not part of the headline line's workload): ``--mode fwd`` runs
only the c1 forward loops (for ``rocprofv3 --pmc`` passes), ``--mode c2`` /
``c3`` / ``c4`` only that configuration's forward+backward loop, and
``--copy-mib N`` first runs one plain device-to-device copy of N MiB, the
calibration kernel whose FETCH_SIZE / WRITE_SIZE readings scale the kernels'
counters.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
REF_README_TFLOPS = 90.2    # reference README.md:14 (RTX 3090, com_2buffer_cpasyc.cu)
METRIC = "DCNv2 fwd TFLOPS (README formula) @B8 C64 128² Co256 3×3 fp16; fwd+bwd ms"
# Forward floors of BASELINE.md section 2 (us): c3 MFMA-bound, c4 HBM/gather-bound.
FWD_FLOOR_US = {"c1_readme_fwd": 15.4, "c3_neck_bf16_dg4": 30.7, "c4_stress_s2_d2": 5.5}
MFMA_STAGES = ("fwd_main", "bwd_colgrad", "bwd_gradw")


def _events_ms(fn, steps, torch):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _median_ms(fn, steps, torch, scrub=None):
    """Median of per-call event times; with `scrub` (a large device buffer)
    every call is preceded by a write of the whole buffer, which evicts the
    L2 and the MALL (256 MB) so the call starts cold."""
    evs = []
    torch.cuda.synchronize()
    for _ in range(steps):
        if scrub is not None:
            scrub.add_(1)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()  # once: the GPU never idles between the calls
    ts = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    return ts[len(ts) // 2]


def _warm(fn, steps, settle_ms, torch):
    """At least `steps` calls and at least `settle_ms` of wall time."""
    n, t0 = 0, time.perf_counter()
    while n < steps or (time.perf_counter() - t0) * 1e3 < settle_ms:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def _stage_avgs(_C, names):
    out = {}
    for s in names:
        ms, n = _C.profile_read(s)
        if n:
            out[s] = ms / n
    return out


COPY_MIB = 512  # calibration copy of the PMC passes


def _pmc_pass(counter, workdir, timeout_s):
    """One ``rocprofv3 --pmc <counter>`` run of ``bench.py --mode fwd`` (c1
    forward loops after one plain device copy of COPY_MIB MiB) as a child
    process.  Returns {kernel name: [counter value per dispatch, KiB]}, or a
    string saying why there is none."""
    import csv
    import glob
    import shutil
    import subprocess
    prof = shutil.which("rocprofv3")
    if not prof:
        return "rocprofv3 not found"
    d = os.path.join(workdir, counter)
    cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "p", "--",
           sys.executable, os.path.join(ROOT, "bench.py"), "--mode", "fwd", "--steps", "3",
           "--warmup", "2", "--settle-ms", "0", "--copy-mib", str(COPY_MIB), "--no-cpu"]
    try:
        # (the profiler may exit non-zero after the program ends with its
        # results complete; the csv decides)
        subprocess.run(cmd, cwd=ROOT, env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                       stderr=subprocess.DEVNULL, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return f"the {counter} pass did not finish in {timeout_s} s"
    except OSError as e:
        return f"the {counter} pass did not start: {e}"
    paths = glob.glob(os.path.join(d, "**", "p_counter_collection.csv"), recursive=True)
    if not paths:
        return f"the {counter} pass wrote no counter file"
    per = {}
    with open(paths[0]) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            key = (r["Kernel_Name"], int(r["Dispatch_Id"]))
            per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    out = {}
    for (name, _), v in per.items():
        out.setdefault(name, []).append(v)
    return out


def _live_traffic(timeout_s=100):
    """HBM bytes per launch of the c1 forward kernel, measured by this run: a
    FETCH_SIZE and a WRITE_SIZE pass (rocprofv3 --pmc, each its own child
    process, run before this process touches the GPU), each reading scaled by
    what the same counter reads for a plain device copy of known size in the
    same pass.  Returns (bytes or None, detail dict)."""
    import statistics
    import tempfile
    detail = {}
    total = 0.0
    with tempfile.TemporaryDirectory(prefix="dcn2_pmc_", dir="/tmp") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            print(f"bench.py: rocprofv3 --pmc {counter} pass over the c1 forward (traffic of its kernel)",
                  file=sys.stderr, flush=True)
            per = _pmc_pass(counter, tmp, timeout_s)
            if isinstance(per, str):
                return None, {"error": per}
            copy = [v for n, vs in per.items() if "copyBuffer" in n for v in vs]
            kern = [v for n, vs in per.items() if "dcn2_fwd_rw_kernel" in n for v in vs]
            if not copy or not kern or max(copy) <= 0:
                return None, {"error": f"the {counter} pass holds no copy or no forward kernel dispatch"}
            factor = COPY_MIB * 1024.0 / max(copy)  # KiB the copy moves / KiB the counter reads
            kib = statistics.median(kern)
            detail[counter] = {"kib_per_launch": round(kib, 1), "copy_factor": round(factor, 4),
                               "dispatches": len(kern)}
            total += kib * factor * 1024.0
    return int(total), detail


def _traffic():
    """HBM bytes per launch of the forward kernel, from the two rocprofv3 PMC
    passes (FETCH_SIZE, WRITE_SIZE) summarised in
    profiles/fwd_kernel_traffic_c1.md (its ``hbm_bytes_per_launch:`` line);
    the fallback when the bench cannot run the passes itself."""
    path = os.path.join(ROOT, "profiles", "fwd_kernel_traffic_c1.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except (OSError, ValueError):
        pass
    return None


def _stage_report(w, stages):
    """Per-stage ms; for the MFMA stages also TFLOP/s and fraction of the dense
    fp16/bf16 (fp32) peak on the algorithmic GEMM FLOPs of one pass.  When the
    backward ran its fused kernel (no ``bwd_gradw`` launch), ``bwd_colgrad``
    holds both backward GEMMs and is credited with twice the FLOPs."""
    import torch
    peak = PEAK_FP32_TFLOPS if w.dtype == torch.float32 else PEAK_FP16_TFLOPS
    fused = "bwd_colgrad" in stages and "bwd_gradw" not in stages
    out = {}
    for k, ms in stages.items():
        e = {"ms": round(ms, 5)}
        if k in MFMA_STAGES:
            gemms = 2 if (fused and k == "bwd_colgrad") else 1
            tf = gemms * w.gemm_flops() / (ms * 1e-3) / 1e12
            e.update(tflops=round(tf, 1), frac=round(tf / peak, 4))
            if gemms == 2:
                e["note"] = "fused kernel: column gradient and grad_weight / grad_bias"
        out[k] = e
    return out


def _geo(w):
    return (w.stride, w.stride, w.pad, w.pad, w.dil, w.dil, w.groups)


def _bwd_workspace_bytes(_C, w, t):
    """dcn2_backward_workspace_bytes of workload w (NCHW tensors t)."""
    import ctypes
    d = _C.make_desc(t["input"], t["weight"], *_geo(w))
    return _C.lib().dcn2_backward_workspace_bytes(ctypes.byref(d))


def cpu_baseline(seconds, threads):
    """The float32 oracle (C, OpenMP) on bounded samples: c1 forward on image
    0 (the metric), c0 forward, and c2 forward + backward on image 0."""
    import torch

    from dcnv2_amd.workloads import CONFIGS, make_inputs
    from oracle import oracle

    def timed(fn, budget):
        fn()  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or reps >= 500:
                return reps, el

    def arrays(w):
        t = make_inputs(w, dtype=torch.float32, with_grad=True)
        return {k: v.numpy() for k, v in t.items()}

    names = ("input", "weight", "mask", "offset", "bias")
    res = {}
    # c1 forward, image 0 (the headline's unit: README-formula TFLOPS)
    c1 = CONFIGS[1].with_(B=1)
    a = arrays(c1)
    r1, e1 = timed(lambda: oracle.dcn_forward(*(a[k] for k in names), **c1.geometry(),
                                              precision="f32", nthreads=threads), seconds * 0.5)
    # c0 forward (the CPU plumbing workload)
    c0 = CONFIGS[0]
    a0 = arrays(c0)
    r0, e0 = timed(lambda: oracle.dcn_forward(*(a0[k] for k in names), **c0.geometry(),
                                              precision="f32", nthreads=threads), seconds * 0.1)
    # c2 forward + backward, image 0
    c2 = CONFIGS[2].with_(B=1)
    a2 = arrays(c2)

    def fb():
        oracle.dcn_forward(*(a2[k] for k in names), **c2.geometry(), precision="f32",
                           nthreads=threads)
        oracle.dcn_backward(*(a2[k] for k in names), a2["grad_output"], **c2.geometry(),
                            precision="f32", nthreads=threads)

    r2, e2 = timed(fb, seconds * 0.4)
    res = {
        "value": c1.readme_flops() * r1 / e1 / 1e12,
        "unit": "TFLOPS (README formula)",
        "cores": threads,
        "kind": "port",
        "sample": f"{r1} x forward of image 0 of c1_readme_fwd (B=1 of 8), float32, {e1:.1f} s; "
                  f"{r0} x c0 forward, {e0:.1f} s; {r2} x forward+backward of image 0 of "
                  f"c2_readme_fwd_bwd, {e2:.1f} s; C oracle with OpenMP",
        "c1_fwd_ms_full_batch": round(e1 / r1 * 1e3 * CONFIGS[1].B, 3),
        "c0_fwd_ms": round(e0 / r0 * 1e3, 4),
        "c2_fwd_bwd_ms_full_batch": round(e2 / r2 * 1e3 * CONFIGS[2].B, 3),
        "os_cpu_count": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "torch_num_threads": torch.get_num_threads(),
        "threads_note": "OpenMP threads of the oracle = OMP_NUM_THREADS when set (the GPU "
                        "box's CPU share per GPU), else the affinity mask; full-batch ms are "
                        "image 0 times the batch",
    }
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=400.0)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", choices=("full", "fwd", "c2", "c3", "c4"), default="full")
    ap.add_argument("--copy-mib", type=int, default=0)
    ap.add_argument("--bwd-slice-mib", type=int, default=0,
                    help="backward workspace budget per slice of images (0: library default)")
    ap.add_argument("--no-live-traffic", action="store_true",
                    help="take roofline.traffic from the committed profile instead of measuring it")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the batch-sharded multi-GPU path is "
              "a design only and is not benchmarked (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    # HBM traffic of the forward kernel: the PMC passes run as child processes
    # first, while this process has not touched the GPU yet
    live_traffic, traffic_detail = (None, {"error": "not measured (--no-live-traffic)"})
    under_profiler = any(k.startswith("ROCPROF_") for k in os.environ) or \
        "rocprofiler" in os.environ.get("LD_PRELOAD", "")
    if under_profiler:
        traffic_detail = {"error": "not measured: this run is itself under a profiler"}
    elif args.mode == "full" and not args.no_live_traffic:
        live_traffic, traffic_detail = _live_traffic()

    import torch

    from dcnv2_amd import _C
    from dcnv2_amd.workloads import CONFIGS, make_inputs

    dev = torch.device("cuda:0")
    c1, c2 = CONFIGS[1], CONFIGS[2]

    def load(w):
        return {k: v.to(dev) for k, v in make_inputs(w, with_grad=True).items()}

    def fwd_fn(w, t):
        args5 = (t["input"], t["weight"], t["mask"], t["offset"], t["bias"])
        return lambda: _C.dcn_v2_forward(*args5, *_geo(w))

    def fwd_bwd_fn(w, t):
        args5 = (t["input"], t["weight"], t["mask"], t["offset"], t["bias"])

        def f():
            _C.dcn_v2_forward(*args5, *_geo(w))
            return _C.dcn_v2_backward(*args5, t["grad_output"], *_geo(w))
        return f

    if args.bwd_slice_mib:
        _C.set_option("bwd_slice_bytes", args.bwd_slice_mib << 20)

    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.mode in ("c2", "c3", "c4"):
        w = CONFIGS[int(args.mode[1])]
        t = load(w)
        f = fwd_bwd_fn(w, t)
        _warm(f, args.warmup, args.settle_ms, torch)
        ms = _events_ms(f, args.steps, torch)
        print(json.dumps({"mode": args.mode, "fwd_bwd_ms": round(ms, 5)}), flush=True)
        return

    t1 = load(c1)
    fwd = fwd_fn(c1, t1)
    warm_run = _warm(fwd, args.warmup, args.settle_ms, torch)
    ms = _events_ms(fwd, args.steps, torch)
    value = c1.readme_flops() / (ms * 1e-3) / 1e12
    # per-call medians: hot (back to back) and cold (512 MiB scrub before each call)
    hot_med = _median_ms(fwd, args.steps, torch)
    scrub = torch.zeros(128 << 20, dtype=torch.float32, device=dev)
    cold_med = _median_ms(fwd, max(10, args.steps // 4), torch, scrub)
    del scrub
    _warm(fwd, 20, 100.0, torch)

    # second loop with per-stage events for the kernel roofline
    _C.profile_enable(True)
    _stage_avgs(_C, _C.STAGES)  # clear
    _events_ms(fwd, args.steps, torch)
    fstages = _stage_avgs(_C, ("fwd_pack", "fwd_main"))
    _C.profile_enable(False)
    kern_ms = fstages["fwd_main"]
    achieved = c1.gemm_flops() / (kern_ms * 1e-3) / 1e12

    if args.mode == "fwd":
        print(json.dumps({"mode": "fwd", "ms_per_step": round(ms, 5),
                          "kernel_ms": round(kern_ms, 5), "fwd_hot_median_ms": round(hot_med, 5),
                          "fwd_cold_median_ms": round(cold_med, 5)}), flush=True)
        return

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOPS (README formula)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_run,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "baseline_note": "no published MI355X number; the reference README's 90.2 README-formula "
                         "TFLOPS (com_2buffer_cpasyc.cu, RTX 3090, README.md:14) is other "
                         "hardware",
        "dtype": "fp16",
        "data": "synthetic (seeded, BASELINE.json config distributions; inputs resident in HBM)",
        "config": {"workload": "c1_readme_fwd: B8 C64 H128 W128 Cout256 3x3 s1 p1 d1 dg1 fp16, "
                               "forward", "global_batch": c1.B, "parallelism": "single GPU"},
        "fwd_real_tflops": round(c1.gemm_flops() / (ms * 1e-3) / 1e12, 2),
        "fwd_hot_median_ms": round(hot_med, 5),
        "fwd_cold_median_ms": round(cold_med, 5),
        "fwd_cold_note": "median per call after a 512 MiB write that evicts L2 and MALL",
        "roofline": {
            "bound": "mfma",
            "kernel": "dcn2_fwd_rw_kernel (weight resident in registers; fused bilinear sampling "
                      "+ 32x32x16 f16 MFMA)",
            "achieved": round(achieved, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": live_traffic if live_traffic is not None else _traffic(),
            "traffic_source": (
                "measured by this run: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, each over "
                "bench.py --mode fwd in a child process, median per dispatch of this kernel scaled "
                f"by the counter's reading for a {COPY_MIB} MiB device copy in the same pass"
                if live_traffic is not None else
                "profiles/fwd_kernel_traffic_c1.md: rocprofv3 FETCH_SIZE + WRITE_SIZE passes of this "
                "kernel, calibrated against a copy of known size (" + traffic_detail["error"] + ")"),
            "traffic_detail": traffic_detail,
            "algorithmic_flops_per_launch": c1.gemm_flops(),
            "kernel_ms": round(kern_ms, 5),
        },
        "stages_ms": {"c1_forward": {k: round(v, 5) for k, v in fstages.items()}},
    }
    del t1

    # forward + backward at the headline shape (c2), and c3 / c4 (forward and
    # forward + backward each), with per-stage times and MFMA fractions
    others = {}
    for w in (c2, CONFIGS[3], CONFIGS[4]):
        t = load(w)
        e = {"workload": f"{w.name}: B{w.B} C{w.C} H{w.H} W{w.W} Cout{w.Cout} {w.k}x{w.k} "
                         f"s{w.stride} p{w.pad} d{w.dil} dg{w.groups} "
                         f"{str(w.dtype).split('.')[-1]}"}
        steps = max(5, args.steps // 4)
        if w is not c2:
            f = fwd_fn(w, t)
            _warm(f, 10, 100.0, torch)
            fms = _events_ms(f, steps, torch)
            _C.profile_enable(True)
            _stage_avgs(_C, _C.STAGES)
            _events_ms(f, steps, torch)
            st = _stage_avgs(_C, ("fwd_pack", "fwd_main"))
            _C.profile_enable(False)
            e["fwd_ms"] = round(fms, 5)
            e["fwd_readme_tflops"] = round(w.readme_flops() / (fms * 1e-3) / 1e12, 1)
            e["fwd_real_tflops"] = round(w.gemm_flops() / (fms * 1e-3) / 1e12, 1)
            e["fwd_stages"] = _stage_report(w, st)
            floor = FWD_FLOOR_US.get(w.name)
            if floor:
                e["fwd_kernel_floor_us"] = floor
                e["fwd_kernel_frac_of_floor"] = round(floor / (st["fwd_main"] * 1e3), 4)
        f = fwd_bwd_fn(w, t)
        _warm(f, 5, 100.0, torch)
        fbms = _events_ms(f, steps, torch)
        _C.profile_enable(True)
        _stage_avgs(_C, _C.STAGES)
        _events_ms(f, steps, torch)
        st = _stage_avgs(_C, _C.STAGES)
        _C.profile_enable(False)
        e["fwd_bwd_ms"] = round(fbms, 5)
        e["bwd_workspace_mb"] = round(_bwd_workspace_bytes(_C, w, t) / 1e6, 1)
        e["fwd_bwd_real_tflops"] = round(3 * w.gemm_flops() / (fbms * 1e-3) / 1e12, 1)
        e["fwd_bwd_stages"] = _stage_report(w, st)
        others[w.name] = e
        del t, f
        torch.cuda.empty_cache()
    result["fwd_bwd_ms"] = others[c2.name]["fwd_bwd_ms"]
    result["configs"] = others

    # Weight groups (torchvision's groups; the reference has none): a layer of
    # the c2 pixel shape with 128 input channels in 2 weight groups, against
    # the same layer ungrouped.  The grouped layer runs one GEMM per group over
    # its own channels, half the sampling and MFMA work of the ungrouped one.
    grp = {}
    for wg in (1, 2):
        w = c2.with_(C=128, seed=7)
        t = load(w)
        if wg > 1:
            t["weight"] = t["weight"][:, : w.C // wg].contiguous()
        f, fb = fwd_fn(w, t), fwd_bwd_fn(w, t)
        _warm(f, 10, 100.0, torch)
        fms = _events_ms(f, max(5, args.steps // 4), torch)
        _warm(fb, 5, 50.0, torch)
        fbms = _events_ms(fb, max(5, args.steps // 4), torch)
        grp[f"weight_groups_{wg}"] = {"fwd_ms": round(fms, 5), "fwd_bwd_ms": round(fbms, 5)}
        del t, f, fb
    result["weight_groups"] = dict(grp, workload="B8 C128 H128 W128 Cout256 3x3 s1 p1 dg1 fp16")

    # The c1/c2 workloads in channels_last: the kernels read the input in
    # place (C = 64 needs no channel padding), so the repacking pass drops out,
    # write the output and grad_input channels-last and read grad_output
    # channels-last, with no layout copy anywhere.
    t2 = load(c2)
    x_cl = t2["input"].to(memory_format=torch.channels_last)
    go_cl = t2["grad_output"].to(memory_format=torch.channels_last)
    b_args = (t2["weight"], t2["mask"], t2["offset"], t2["bias"])

    def fwd_cl():
        return _C.dcn_v2_forward(x_cl, *b_args, *_geo(c1))

    def fwd_bwd_cl():
        _C.dcn_v2_forward(x_cl, *b_args, *_geo(c2))
        return _C.dcn_v2_backward(x_cl, *b_args, go_cl, *_geo(c2))

    fb_steps = max(5, args.steps // 4)
    _warm(fwd_cl, 20, 100.0, torch)
    cl_fwd_ms = _events_ms(fwd_cl, args.steps, torch)
    _warm(fwd_bwd_cl, 5, 50.0, torch)
    result["channels_last"] = {
        "fwd_ms": round(cl_fwd_ms, 5),
        "fwd_readme_tflops": round(c1.readme_flops() / (cl_fwd_ms * 1e-3) / 1e12, 2),
        "fwd_bwd_ms": round(_events_ms(fwd_bwd_cl, fb_steps, torch), 5),
        "note": "input, output, grad_output and grad_input channels_last, all read or written "
                "in place",
    }
    del x_cl, go_cl

    # The DCN module (offset/mask predictor conv + operator) at the same shape,
    # forward + backward: the fused path hands the predictor output to the
    # kernels; the separate path materialises chunk / cat / sigmoid as the
    # reference's DCN.forward does (dcn_v2_mm.py:133-137).
    from dcnv2_amd.dcn_v2_mm import DCN
    mod_ms = {}
    x = t2["input"].clone().requires_grad_(True)
    for fused in (True, False):
        torch.manual_seed(0)
        mod = DCN(c2.C, c2.Cout, c2.k, c2.stride, c2.pad, c2.dil, c2.groups,
                  fused_offset_mask=fused).to(dev).half()
        with torch.no_grad():
            mod.conv_offset_mask.weight.normal_(0.0, 0.01)

        def module_step():
            y = mod(x)
            y.backward(t2["grad_output"])

        _warm(module_step, 5, 50.0, torch)
        mod_ms["fused" if fused else "separate"] = round(_events_ms(module_step, fb_steps, torch), 5)
    result["dcn_module_fwd_bwd_ms"] = dict(mod_ms, workload="DCN module (predictor conv + "
                                           "operator), c2 shape, fp16, forward + backward")
    del t2, x
    if not args.no_cpu:
        omp = os.environ.get("OMP_NUM_THREADS", "")
        threads = int(omp) if omp.isdigit() and int(omp) > 0 else len(os.sched_getaffinity(0))
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, threads)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
