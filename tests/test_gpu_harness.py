"""The C++ harness (tests/harness/bench_flash_attention.cpp), a consumer of
include/flash_attention.h in the shape of the reference's study harness
(benchmarks/bench_flash_attention.cu:391-731), run on the GPU in --quick
mode: its accuracy suite must pass both gates for every supported kernel, its
timed outputs must be finite, and its three CSV files must carry the
reference's column sets (:419-424), so the reference's plotting reads them.
"""
import csv
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "harness", "bench_flash_attention")

RAW = "kernel,batch,heads,seq_len,head_dim,causal,iteration,elapsed_ms".split(",")
SUMMARY = ("kernel,batch,heads,seq_len,head_dim,causal,status,warmup_iters,timed_iters,median_ms,q1_ms,q3_ms,"
           "iqr_ms,baseline_median_ms,speedup_vs_v0,tflops,algorithmic_hbm_gb,v0_workspace_bytes,output_nan,"
           "output_inf").split(",")
ACCURACY = ("kernel,batch,heads,seq_len,head_dim,causal,vs_double,row_scaled_error,max_abs_error,row_scale_ulp,"
            "output_nan,output_inf,reference_nan,reference_inf,passed").split(",")


def rows(path):
    with open(path, newline="") as fh:
        reader = csv.DictReader(fh)
        return reader.fieldnames, list(reader)


def test_harness_quick(tmp_path):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is missing: run __graft_entry__.build()")
    print("harness --quick", flush=True)
    run = subprocess.run([BINARY, "--quick", str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-2000:]

    fields, acc = rows(tmp_path / "accuracy.csv")
    assert fields[:len(ACCURACY)] == ACCURACY and fields[-1] == "abs_gate"
    kernels = {r["kernel"] for r in acc}
    assert kernels == {"v0_unfused", "v3_tensorcore", "v3b_tensorcore"}
    assert len(acc) == 3 * 2 * 2  # kernels x head_dim x mask
    for r in acc:
        assert r["passed"] == "1" and float(r["row_scale_ulp"]) <= 2.0 and float(r["abs_gate"]) <= 1.0, r

    fields, summ = rows(tmp_path / "summary.csv")
    assert fields == SUMMARY
    assert len(summ) == 8 * 6  # 8 quick cases x 6 entries
    for r in summ:
        if r["kernel"] in ("v1_fused_row", "v2a_fused_tiled", "v2b_fused_tiled"):
            assert r["status"] == "unsupported"
            continue
        assert r["status"] == "ok" and r["output_nan"] == "0" and r["output_inf"] == "0", r
        q1, med, q3 = float(r["q1_ms"]), float(r["median_ms"]), float(r["q3_ms"])
        assert 0 < q1 <= med <= q3
        if r["kernel"] != "v0_unfused":
            assert float(r["speedup_vs_v0"]) > 1.0, r

    fields, raw = rows(tmp_path / "raw_timings.csv")
    assert fields == RAW
    assert len(raw) == 8 * 3 * 30


def test_v0_profile_modes(tmp_path):
    """The v0 stage profile's other two modes (benchmarks/profile_attention_v0.cu:
    195-197): one shape with its own sample and warmup counts (a stage-timing
    CSV with the reference's columns and five metrics), and the profiler mode
    (plain instrumented launches without events or checks, for rocprofv3)."""
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is missing: run __graft_entry__.build()")
    print("harness --v0-profile shape", flush=True)
    run = subprocess.run([BINARY, "--v0-profile", "1", "2", "300", "64", "1", "4", "1", str(tmp_path)],
                         capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-2000:]
    assert "PASS (finite, bitwise equal to v0)" in run.stdout
    fields, stage = rows(tmp_path / "v0_stage_timing.csv")
    assert fields == ("shape,batch,heads,seq_len,head_dim,causal,metric,median_ms,q1_ms,q3_ms,iqr_ms,"
                      "share_of_pipeline").split(",")
    assert [r["metric"] for r in stage] == ["QK", "softmax", "PV", "instrumented_pipeline", "original_v0_e2e"]
    assert all(r["shape"] == "b1h2n300d64_causal" and float(r["median_ms"]) > 0 for r in stage)

    print("harness --v0-profile --profiler", flush=True)
    run = subprocess.run([BINARY, "--v0-profile", "--profiler", "1", "2", "300", "64", "0", "3"],
                         capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-2000:]
    assert "3 iteration(s), output finite" in run.stdout
    bad = subprocess.run([BINARY, "--v0-profile", "--profiler"], capture_output=True, text=True, timeout=60)
    assert bad.returncode == 2


def test_grid_goes_on_when_v0_workspace_fails(tmp_path):
    """The reference's out-of-memory path (benchmarks/bench_flash_attention.cu:
    614-629,655-667), forced with --workspace-cap=0: every grid case's v0
    allocation "fails", v0 is skipped with status workspace_allocation_failed
    and the run goes on, timing the fused kernels of every case (without a
    speed-up, since there is no baseline)."""
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is missing: run __graft_entry__.build()")
    print("harness --quick --workspace-cap=0", flush=True)
    run = subprocess.run([BINARY, "--quick", "--workspace-cap=0", str(tmp_path)], capture_output=True, text=True,
                         timeout=300)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-2000:]
    assert run.stderr.count("V0 workspace allocation failed") == 8
    fields, summ = rows(tmp_path / "summary.csv")
    assert fields == SUMMARY and len(summ) == 8 * 6
    for r in summ:
        if r["kernel"] == "v0_unfused":
            assert r["status"] == "workspace_allocation_failed" and r["median_ms"] == "", r
            assert int(r["v0_workspace_bytes"]) == 8 * int(r["seq_len"]) ** 2 * 4
        elif r["kernel"] in ("v3_tensorcore", "v3b_tensorcore"):
            assert r["status"] == "ok" and float(r["median_ms"]) > 0 and r["speedup_vs_v0"] == "", r
        else:
            assert r["status"] == "unsupported"
    assert "48 kernel/shape runs skipped" not in run.stdout  # the fused rows did run
    assert "32 kernel/shape runs skipped" in run.stdout       # 8 x (v0 + v1 + v2a + v2b)
