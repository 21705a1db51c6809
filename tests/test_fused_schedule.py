"""CPU check of the fused kernel's barrier schedule (csrc/fa_fused_schedule.hpp).

The kernel's two wave groups must execute exactly the same number of
workgroup barriers or the workgroup deadlocks. The header holds the phase walk
the kernel itself runs (fused_group_walk); this test compiles that header with
g++, drives the walk with counting callbacks, and checks for every tile count
that (a) the walk performs fused_group_barriers() barriers, (b) the stage
parity argument equals kk % 2, and (c) after padding both groups reach the
same total, split.barriers.
"""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "cuda_fused_attention_amd", "csrc")

PROGRAM = r'''
#include "fa_fused_schedule.hpp"
#include <cstdio>
int main() {
    long bad = 0;
    for (int n_tiles = 1; n_tiles <= 20000; ++n_tiles) {
        const fa::FusedSplit sp = fa::fused_split(n_tiles);
        if (sp.count0 + sp.count1 != n_tiles || sp.count0 < sp.count1 || sp.first1 != sp.count0) ++bad;
        for (int g = 0; g < 2; ++g) {
            const int cnt = g == 0 ? sp.count0 : sp.count1;
            int barriers = 1 + (g == 1 ? 1 : 0);   // prologue, group 1's idle phase
            int mfma = 0, valu = 0;
            fa::fused_group_walk(cnt,
                [&](auto par, int kk) { ++barriers; ++mfma; if (decltype(par)::value != kk % 2 || kk > cnt) ++bad; },
                [&](auto par, int kk) { ++barriers; ++valu; if (decltype(par)::value != kk % 2 || kk >= cnt) ++bad; });
            if (mfma != cnt + 1 || valu != cnt) ++bad;
            if (barriers != fa::fused_group_barriers(g, cnt)) ++bad;
            if (barriers > sp.barriers) ++bad;       // padding cannot be negative
        }
    }
    std::printf("%ld\n", bad);
    return bad != 0;
}
'''


def test_barrier_schedule_matches_for_both_groups(tmp_path):
    src = tmp_path / "sched.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "sched"
    r = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout + out.stderr
