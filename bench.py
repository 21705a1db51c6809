#!/usr/bin/env python3
"""Benchmark of the MI355X BF16 attention forward (one GPU).

Metric: BF16 attention-forward TFLOP/s and % of MI355X dense
BF16 MFMA peak at (2,8,2048,D=64/128), dense/causal. A "step" is one fused
forward launch over one batch of synthetic input resident in HBM. The
headline workload is BASELINE config 2, (2,8,2048,64) dense; the other three
(2,8,2048,D) cases, the HIP v0 baseline and its HBM roofline ride along in
"shapes" and "v0". FLOPs follow BASELINE: 4*B*H*N^2*D, halved for causal.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints ONE JSON line. Order: the per-shape extras for the four (2,8,2048,D)
cases (median/IQR of 5 warmups + 30 individually timed launches per kernel,
benchmarks/bench_flash_attention.cu:265-299; then, after a clock ramp, the
average of back-to-back launches between one event pair for v3 and v0, with
the fraction of peak and the speed-up over v0 under both timings; and the v0
per-stage medians, benchmarks/profile_attention_v0.cu:141-190), then a clock ramp
(untimed launches of the measured kernel for --ramp-s seconds: the GPU's
clock takes a few hundred milliseconds of load to settle, and a cold start
reads up to 10 % slow), then W untimed warmup launches, a synchronisation, and
K launches bracketed by hipEvents recorded on the launch stream (inside the
library, fa_time_batch) and by host synchronisation. `value` is the whole-job
rate over that region, `roofline.achieved` the same FLOPs over the average
launch duration from the events. After the timed region a calibration
kernel measures the dense bf16 matrix rate this box sustains under full MFMA
load (fa_mfma_peak); `roofline.frac` stays against the published 2.5 PFLOP/s
and `roofline.frac_of_sustained` divides by that same-run rate, so a change of
a point or two can be told apart from box-to-box clock spread. Inputs come from the package's seeded
generator (cuda_fused_attention_amd/inputs.py); only the cpu_baseline leg
loads the oracle.
"""
from __future__ import annotations

import argparse
import hashlib
import re
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense BF16 MFMA (published)
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E (published)
METRIC = "BF16 attn fwd TFLOP/s + % MFMA peak at (2,8,2048,D=64/128) dense/causal"
WORKLOADS = {
    "c2": (2, 8, 2048, 64, False),
    "c2_causal": (2, 8, 2048, 64, True),
    "headline": (2, 8, 2048, 128, False),
    "c3": (2, 8, 2048, 128, True),
    "c5": (1, 16, 16384, 128, True),
}
# Input family per workload: BASELINE's uniform[-1,1), or its long-sequence
# stress family for c5 (Q, K ~ N(0, 3^2), V uniform).
FAMILY = {"c5": "stress"}
# The per-shape extras (v3, v3b and v0 medians) cover BASELINE's four
# (2,8,2048,D) shapes.
EXTRA_WORKLOADS = ("c2", "c2_causal", "headline", "c3")
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
# The sources that define the fused kernel's code: profiles/traffic.json
# records their hash next to each counter measurement, and a measurement
# taken on other code is reported as stale (traffic null). The hash covers
# the C++ sources with their comments removed and the device compiler flags,
# so a change to comments alone keeps a measurement valid.
KERNEL_SOURCES = ("cuda_fused_attention_amd/csrc/fa_fused.hip", "cuda_fused_attention_amd/csrc/fa_fused_schedule.hpp",
                  "cuda_fused_attention_amd/csrc/fa_common.hpp")


def strip_cpp_comments(text: str) -> str:
    """C++ source without // and /* */ comments and with each line's
    surrounding whitespace and the blank lines dropped (the kernel sources
    hold no string literal with comment markers)."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return "\n".join(line.strip() for line in text.splitlines() if line.strip())


def kernel_source_sha() -> str:
    from cuda_fused_attention_amd import _build

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), encoding="utf-8") as fh:
            h.update(rel.encode() + b"\0" + strip_cpp_comments(fh.read()).encode() + b"\0")
    h.update(repr(_build.HIP_FLAGS).encode())
    return h.hexdigest()[:16]


def baseline_flops(B, H, N, D, causal):
    f = 4.0 * B * H * N * N * D
    return f / 2.0 if causal else f


def make_device_inputs(B, H, N, D, family="uniform"):
    from cuda_fused_attention_amd import inputs

    make = inputs.make_stress_inputs if family == "stress" else inputs.make_uniform_inputs
    host = make(B, H, N, D)
    return host, [inputs.to_device(x) for x in host]


def measure_shape(fa, dev, B, H, N, D, causal, kernel, ws=None):
    import torch

    shape = fa.AttentionShape(B, H, N, D)
    o = torch.empty_like(dev[0])
    samples = fa.time_launches(kernel, *dev, o, ws, shape, causal, warmup=5, iters=30)
    summ = fa.summarize(samples)
    flops = baseline_flops(B, H, N, D, causal)
    out = {
        "median_ms": summ["median_ms"],
        "iqr_ms": summ["iqr_ms"],
        "tflops": flops / (summ["median_ms"] * 1e-3) / 1e12,
    }
    out["pct_peak"] = 100.0 * out["tflops"] / PEAK_BF16_TFLOPS
    return out


def cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host_inputs, B, H, N, D, causal):
    """The FP64 oracle (a C++ port of benchmarks/bench_flash_attention.cu:105-145)
    timed on this host: all rows of the workload on up to 16 threads (the GPU
    box's CPU share), plus one slab on 1 thread (the reference's semantics).
    For seq_len > 2048 it times a stratified row sample instead (every 8th row
    of every slab; every 64th of slab 0 for the single thread) and
    extrapolates the whole-workload time linearly in (row, key) pairs, as the
    sample string says."""
    import numpy as np

    import oracle

    q, k, v = host_inputs
    threads = max(1, min(16, os.cpu_count() or 1))
    flops = baseline_flops(B, H, N, D, causal)
    if N > 2048:
        return cpu_baseline_sampled(host_inputs, B, H, N, D, causal, threads, flops)

    def repeat(fn, min_s):
        runs, t0 = 0, time.perf_counter()
        while True:
            fn()
            runs += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= min_s:
                return runs, elapsed

    runs_all, t_all = repeat(lambda: oracle.attention(q, k, v, causal, threads=threads), 10.0)
    rows1 = np.arange(N, dtype=np.int64)  # slab 0 only
    runs_one, t_one = repeat(lambda: oracle.attention(q, k, v, causal, rows=rows1, threads=1), 3.0)
    return {
        "value": runs_all * flops / t_all / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"whole workload ({B * H * N} rows of ({B},{H},{N},{D}) {'causal' if causal else 'dense'}) "
                  f"on {threads} threads, {runs_all} runs in {t_all:.1f} s",
        "single_thread": {"value": runs_one * flops / (B * H) / t_one / 1e12, "unit": "TFLOP/s",
                          "sample": f"slab 0 ({N} rows) on 1 thread, {runs_one} runs in {t_one:.1f} s"},
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model(),
    }


def cpu_baseline_sampled(host_inputs, B, H, N, D, causal, threads, flops):
    import numpy as np

    import oracle

    q, k, v = host_inputs

    def pairs(rows_in_slab):
        return float(np.sum(rows_in_slab + 1)) if causal else float(len(rows_in_slab)) * N

    def timed(rows, min_s):
        runs, t0 = 0, time.perf_counter()
        while True:
            oracle.attention(q, k, v, causal, rows=rows, threads=threads)
            runs += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= min_s:
                return runs, elapsed

    total_pairs = pairs(np.arange(N)) * B * H
    strided = np.arange(0, N, 8, dtype=np.int64)
    rows_all = (np.arange(B * H, dtype=np.int64)[:, None] * N + strided[None, :]).ravel()
    runs_all, t_all = timed(rows_all, 10.0)
    est_all = t_all / runs_all * total_pairs / (pairs(strided) * B * H)
    strided1 = np.arange(0, N, 64, dtype=np.int64)
    runs_one, t_one = 0, time.perf_counter()
    while True:
        oracle.attention(q, k, v, causal, rows=strided1, threads=1)
        runs_one += 1
        if time.perf_counter() - t_one >= 3.0:
            break
    t_one = time.perf_counter() - t_one
    est_one = t_one / runs_one * pairs(np.arange(N)) / pairs(strided1)
    return {
        "value": flops / est_all / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"every 8th row of all {B * H} slabs of ({B},{H},{N},{D}) {'causal' if causal else 'dense'} "
                  f"on {threads} threads, {runs_all} runs in {t_all:.1f} s; whole-workload time "
                  f"extrapolated linearly in (row, key) pairs: {est_all:.1f} s",
        "single_thread": {"value": flops / (B * H) / est_one / 1e12, "unit": "TFLOP/s",
                          "sample": f"every 64th row of slab 0 on 1 thread, {runs_one} runs in {t_one:.1f} s; "
                                    f"one slab extrapolated to {est_one:.1f} s"},
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model(),
    }


def load_traffic(key):
    """(HBM bytes per launch, status) from profiles/traffic.json for this
    kernel:workload; None unless it was measured on the current kernel sources."""
    try:
        with open(TRAFFIC_FILE) as fh:
            entry = json.load(fh).get(key)
    except (OSError, ValueError):
        return None, "no traffic.json"
    if not entry:
        return None, f"no measurement for {key}"
    if entry.get("kernel_source_sha") != kernel_source_sha():
        return None, "stale: measured on other kernel sources"
    return entry.get("hbm_bytes_per_launch"), f"rocprofv3 FETCH_SIZE/WRITE_SIZE, {entry.get('source')}"


def measure_back_to_back(fa, dev, B, H, N, D, causal, kernel, ws=None, min_s=0.15, ramp_s=0.2):
    """Average launch time (ms) of back-to-back launches between one event
    pair (fa_time_batch), after `ramp_s` seconds of untimed launches, over
    enough launches for about `min_s` seconds."""
    import torch

    shape = fa.AttentionShape(B, H, N, D)
    o = torch.empty_like(dev[0])
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < ramp_s:
        fa.time_batch(kernel, *dev, o, ws, shape, causal, iters=20)
    probe = fa.time_batch(kernel, *dev, o, ws, shape, causal, iters=20) / 20
    iters = max(20, int(min_s * 1e3 / max(probe, 1e-3)))
    return fa.time_batch(kernel, *dev, o, ws, shape, causal, iters=iters) / iters, iters


def v0_stage_timing(fa, dev, B, H, N, D, causal, iters=30, warmup=5):
    """benchmarks/profile_attention_v0.cu:141-190: per-stage milliseconds of
    the instrumented v0 launch (QK, softmax, PV and total), median and IQR
    over `iters` launches, each synchronised."""
    import torch

    shape = fa.AttentionShape(B, H, N, D)
    ws = torch.empty(fa.unfused_workspace_bytes(shape) // 4, dtype=torch.float32, device="cuda")
    o = torch.empty_like(dev[0])
    events = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    samples = {"qk": [], "softmax": [], "pv": [], "total": []}
    for it in range(warmup + iters):
        fa.launch_attention_unfused_profile(*dev, o, ws, shape, causal, events=events)
        torch.cuda.synchronize()
        if it < warmup:
            continue
        t = [events[i].elapsed_time(events[i + 1]) for i in range(3)]
        for name, val in zip(("qk", "softmax", "pv"), t):
            samples[name].append(val)
        samples["total"].append(events[0].elapsed_time(events[3]))
    out = {"shape": [B, H, N, D], "causal": causal, "timed_iters": iters}
    for name, xs in samples.items():
        summ = fa.summarize(xs)
        out[name] = {"median_ms": summ["median_ms"], "iqr_ms": summ["iqr_ms"]}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--ramp-s", type=float, default=0.3, help="seconds of untimed launches before the warmup")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    ap.add_argument("--kernel", choices=["v3_mfma", "v3b_mfma", "v0_unfused"], default="v3_mfma",
                    help="kernel in the timed region (v0_unfused: the three-kernel baseline, HBM roofline)")
    ap.add_argument("--no-extras", action="store_true", help="only the timed region (for profiling runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-calibration", action="store_true", help="skip the sustained-MFMA-rate calibration")
    ap.add_argument("--family", choices=["uniform", "stress"], default=None,
                    help="input family (default: the workload's own: stress for c5, uniform otherwise)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run a plain elementwise copy of this many MiB (rocprof counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the attention "
              "forward has no multi-GPU path here — run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0 or args.warmup < 0:
        sys.exit("steps must be > 0 and warmup >= 0")

    import torch

    import cuda_fused_attention_amd as fa

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)

    B, H, N, D, causal = WORKLOADS[args.workload]
    family = args.family or FAMILY.get(args.workload, "uniform")
    host_inputs, dev = make_device_inputs(B, H, N, D, family)
    shape = fa.AttentionShape(B, H, N, D)
    o = torch.empty_like(dev[0])
    flops = baseline_flops(B, H, N, D, causal)
    stream = torch.cuda.current_stream()
    timed_ws = None
    if args.kernel == "v0_unfused":
        timed_ws = torch.empty(fa.unfused_workspace_bytes(shape) // 4, dtype=torch.float32, device="cuda")

    shapes = None
    if not args.no_extras:
        shapes = {}
        for name in EXTRA_WORKLOADS:
            b, h, n, d, c = WORKLOADS[name]
            same = (b, h, n, d) == (B, H, N, D) and family == "uniform"
            _, sdev = (None, dev) if same else make_device_inputs(b, h, n, d)
            sh = fa.AttentionShape(b, h, n, d)
            entry = {"shape": [b, h, n, d], "causal": c}
            for kern in ("v3_mfma", "v3b_mfma"):
                entry[kern] = measure_shape(fa, sdev, b, h, n, d, c, kern)
            ws = torch.empty(fa.unfused_workspace_bytes(sh) // 4, dtype=torch.float32, device="cuda")
            v0 = measure_shape(fa, sdev, b, h, n, d, c, "v0_unfused", ws)
            v0_bytes = 16.0 * b * h * n * n + 8.0 * b * h * n * d
            v0["hbm_gbps"] = v0_bytes / (v0["median_ms"] * 1e-3) / 1e9
            v0["hbm_frac"] = v0["hbm_gbps"] / PEAK_HBM_GBPS
            v0["algorithmic_bytes"] = v0_bytes
            v0["reference_model_bytes"] = 20.0 * b * h * n * n + 8.0 * b * h * n * d
            entry["v0_unfused"] = v0
            entry["v3_config"] = dict(zip(("rows_per_block", "kv_groups"), fa.tensorcore_v3_config(sh, c)))
            # Back-to-back: the kernel's own duration, without the ~7 us of
            # idle-queue dispatch each individually timed launch carries.
            flops_s = baseline_flops(b, h, n, d, c)
            b2b_ms, b2b_iters = measure_back_to_back(fa, sdev, b, h, n, d, c, "v3_mfma")
            entry["v3_mfma"].update({"b2b_ms": b2b_ms, "b2b_launches": b2b_iters,
                                     "b2b_tflops": flops_s / (b2b_ms * 1e-3) / 1e12,
                                     "b2b_frac": flops_s / (b2b_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS})
            v0_b2b_ms, v0_iters = measure_back_to_back(fa, sdev, b, h, n, d, c, "v0_unfused", ws, min_s=0.1,
                                                       ramp_s=0.05)
            v0.update({"b2b_ms": v0_b2b_ms, "b2b_launches": v0_iters,
                       "b2b_hbm_gbps": v0_bytes / (v0_b2b_ms * 1e-3) / 1e9})
            entry["speedup_vs_v0"] = v0["median_ms"] / entry["v3_mfma"]["median_ms"]
            entry["speedup_vs_v0_b2b"] = v0_b2b_ms / b2b_ms
            shapes[name] = entry
            del ws, sdev
        # v0 per-stage record at the reference's profiling shape (c2)
        b, h, n, d, c = WORKLOADS["c2"]
        _, sdev = make_device_inputs(b, h, n, d)
        v0_stages = v0_stage_timing(fa, sdev, b, h, n, d, c)
        del sdev
        torch.cuda.synchronize()

    # Clock ramp: untimed launches until --ramp-s seconds have passed.
    ramp_launches = 0
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < args.ramp_s:
        fa.time_batch(args.kernel, *dev, o, timed_ws, shape, causal, iters=50, stream=stream)
        ramp_launches += 50
    # W untimed warmup launches, then the timed region: K launches bracketed
    # by synchronisation (wall clock) and by hipEvents on the launch stream.
    if args.warmup:
        fa.time_batch(args.kernel, *dev, o, timed_ws, shape, causal, iters=args.warmup, stream=stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    event_ms = fa.time_batch(args.kernel, *dev, o, timed_ws, shape, causal, iters=args.steps, stream=stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0

    value = args.steps * flops / wall_s / 1e12
    avg_launch_ms = event_ms / args.steps
    achieved = flops / (avg_launch_ms * 1e-3) / 1e12

    # Same-run calibration of the sustained matrix rate (after the timed
    # region: its full-MFMA load lowers the clock): every wave of two per
    # SIMD issuing back-to-back MFMAs on operands drawn from this workload's
    # own Q (the clock under full MFMA load depends on the data: zeros hold
    # 2.4 GHz, uniform[-1,1) about 1.94 GHz, N(0, 3^2) about 1.76 GHz);
    # ~0.3 ms per launch. A 50-launch run lets the clock settle (it takes
    # tens of milliseconds of this load), then three runs of 20 launches:
    # their median, all three reported.
    calib, calib_runs = None, []
    if not args.no_calibration:
        fa.mfma_peak(mfma_per_wave=8192, launches=50, operands=dev[0], stream=stream)
        calib_runs = [fa.mfma_peak(mfma_per_wave=8192, launches=20, operands=dev[0], stream=stream)
                      for _ in range(3)]
        calib = sorted(calib_runs, key=lambda r: r["tflops"])[1]

    if args.calib_copy_mib:
        x = torch.ones(args.calib_copy_mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        torch.neg(x, out=y)
        torch.cuda.synchronize()

    traffic, traffic_source = load_traffic(f"{args.kernel}:{args.workload}")
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall_s * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: Q/K ~ N(0, 3^2) (Box-Muller) and V uniform[-1,1), rounded to bf16, SplitMix64 "
                 "seeds 11/22/33, resident in HBM" if family == "stress" else
                 "synthetic: Q/K/V uniform[-1,1) rounded to bf16, SplitMix64 seeds 11/22/33, resident in HBM"),
        "config": {
            "workload": f"{args.workload}: fused attention forward ({B},{H},{N},{D}) "
                        f"{'causal' if causal else 'dense'}, [B,H,N,D] bf16, fp32 accumulate",
            "batch": B, "heads": H, "seq_len": N, "head_dim": D, "causal": causal, "kernel": args.kernel,
            "flops_per_step": flops, "flop_convention": "4*B*H*N^2*D, halved for causal (BASELINE)",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 5),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "avg_launch_us": avg_launch_ms * 1e3,
            "algorithmic_flops_per_launch": flops,
            "min_hbm_bytes_per_launch": 8.0 * B * H * N * D,
        },
        "device": {"name": props.name, "compute_units": props.multi_processor_count,
                   "gcn_arch": getattr(props, "gcnArchName", "")},
    }

    if args.kernel == "v0_unfused":
        # The baseline is bounded by HBM: algorithmic bytes = S written once,
        # read and written once by the softmax, read once by PV, plus Q,K,V,O.
        v0_bytes = 16.0 * B * H * N * N + 8.0 * B * H * N * D
        gbps = v0_bytes / (avg_launch_ms * 1e-3) / 1e9
        result["roofline"].update({"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                   "frac": round(gbps / PEAK_HBM_GBPS, 5), "algorithmic_bytes_per_launch": v0_bytes,
                                   "bytes_model": "16*B*H*N^2 + 8*B*H*N*D (three kernels per launch)"})
    if calib is not None and args.kernel != "v0_unfused":
        # frac stays against the published peak; frac_of_sustained divides by
        # what this box's matrix pipes sustained in this process.
        result["roofline"].update({
            "sustained_peak": round(calib["tflops"], 3),
            "frac_of_sustained": round(achieved / calib["tflops"], 5),
            "sustained_clock_ghz": round(calib["clock_ghz"], 4),
            "sustained_source": f"fa_mfma_peak: one 512-thread workgroup per CU, {calib['mfma_per_wave']} "
                                "back-to-back v_mfma_f32_32x32x16_bf16 per wave on operands taken from this "
                                f"workload's Q ({family}), median of 3 x {calib['launches']} launches after a "
                                "50-launch settle",
            "sustained_runs": [{"tflops": round(r["tflops"], 1), "clock_ghz": round(r["clock_ghz"], 4)}
                               for r in calib_runs],
        })
        if shapes is not None:
            for entry in shapes.values():
                entry["v3_mfma"]["b2b_frac_of_sustained"] = entry["v3_mfma"]["b2b_tflops"] / calib["tflops"]
    result["clock_ramp_launches"] = ramp_launches
    if shapes is not None:
        result["shapes"] = shapes
        result["v0_stages"] = v0_stages
        if args.workload in shapes:
            result["v0"] = {"bound": "hbm", "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                            "achieved": shapes[args.workload]["v0_unfused"]["hbm_gbps"],
                            "frac": shapes[args.workload]["v0_unfused"]["hbm_frac"],
                            "bytes_model": "16*B*H*N^2 + 8*B*H*N*D"}

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(host_inputs, B, H, N, D, causal)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
