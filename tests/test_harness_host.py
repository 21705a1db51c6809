"""CPU tests of the C++ harness's host logic (tests/harness/bench_flash_attention.cpp),
compiled without its main and linked with the libraries; no kernel runs.

The reference keeps timing the grid when v0's score workspace cannot be
allocated: the allocation failure is recoverable, v0's summary row says
"workspace_allocation_failed", and the fused kernels of that case and the
later cases still run (benchmarks/bench_flash_attention.cu:614-629,655-667).
Here the harness's allocation is forced to fail with its byte cap
(--workspace-cap), so no device is needed.
"""
import csv
import io
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"

PROGRAM = r'''
#define FA_HARNESS_NO_MAIN
#include "bench_flash_attention.cpp"
#include <sstream>
int main()
{
    const fa::AttentionShape s{4, 8, 8192, 64};
    const size_t bytes = fa::unfused_workspace_bytes(s);
    // above the cap: the out-of-memory path, without touching a device
    if (allocate_workspace(bytes, bytes - 1, s) != nullptr) return 3;
    std::ostringstream rows;
    int ran = 0;
    for (const Entry& e : entries())
    {
        const char* why = skip_reason(e.supported(64), e.needs_workspace, false);
        if (why) write_skip_row(rows, e.name, s, true, why, e.hbm_bytes(s, true) / 1e9, bytes);
        else std::printf("runs %s\n", e.name), ++ran;
    }
    std::printf("%s", rows.str().c_str());
    return ran == 2 ? 0 : 5;
}
'''


@pytest.fixture(scope="module")
def harness_host(tmp_path_factory, fa_lib, oracle_mod):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("harness_host")
    src = d / "host_check.cpp"
    src.write_text(PROGRAM)
    exe = d / "host_check"
    pkg = os.path.dirname(fa_lib.LIB_PATH)
    odir = os.path.join(REPO, "oracle")
    subprocess.run([HIPCC, "-std=c++17", "-O1", f"-I{REPO}/include", f"-I{odir}", f"-I{REPO}/tests/harness", str(src),
                    "-o", str(exe), f"-L{pkg}", "-lfa_mi355x", f"-L{odir}", "-loracle",
                    f"-Wl,-rpath,{pkg}:{odir}"], check=True, capture_output=True)
    return exe


def test_workspace_allocation_failure_skips_v0_only(harness_host):
    run = subprocess.run([str(harness_host)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    # the reference's note on stderr
    assert "V0 workspace allocation failed: B=4 H=8 N=8192 D=64, 8192.0 MiB." in run.stderr
    # the fused kernels of the case still run
    assert [l for l in run.stdout.splitlines() if l.startswith("runs ")] == ["runs v3_tensorcore",
                                                                          "runs v3b_tensorcore"]
    lines = [l for l in run.stdout.splitlines() if not l.startswith("runs ")]
    header = ("kernel,batch,heads,seq_len,head_dim,causal,status,warmup_iters,timed_iters,median_ms,q1_ms,q3_ms,"
              "iqr_ms,baseline_median_ms,speedup_vs_v0,tflops,algorithmic_hbm_gb,v0_workspace_bytes,output_nan,"
              "output_inf")
    rows = list(csv.DictReader(io.StringIO(header + "\n" + "\n".join(lines) + "\n")))
    status = {r["kernel"]: r["status"] for r in rows}
    assert status == {"v0_unfused": "workspace_allocation_failed", "v1_fused_row": "unsupported",
                      "v2a_fused_tiled": "unsupported", "v2b_fused_tiled": "unsupported"}
    v0 = next(r for r in rows if r["kernel"] == "v0_unfused")
    assert (v0["batch"], v0["heads"], v0["seq_len"], v0["head_dim"], v0["causal"]) == ("4", "8", "8192", "64", "1")
    assert v0["warmup_iters"] == "0" and v0["timed_iters"] == "0" and v0["median_ms"] == ""
    assert int(v0["v0_workspace_bytes"]) == 4 * 8 * 8192 * 8192 * 4
    # the reference's five-pass model: Q, K, V, O once plus 20 bytes per score
    assert float(v0["algorithmic_hbm_gb"]) == pytest.approx((8 * 4 * 8 * 8192 * 64 + 20 * 4 * 8 * 8192 ** 2) / 1e9)
