"""CPU check of the fused kernel's tile / stage / barrier schedule
(csrc/fa_fused_schedule.hpp).

The kernel's wave groups (one, two or four) must execute exactly the same
number of workgroup barriers or the workgroup deadlocks, and the LDS stage rotation must
never overwrite a tile that a later step still reads. The header holds the
walk the kernel itself runs (fused_group_walk) and the pipeline distances; this
test compiles it with g++, replays the walk with a model of the kernel's
per-step actions and checks, for every tile count:
  (a) the walk performs fused_group_barriers() barriers and the compile-time
      step argument equals jj % kFusedUnroll;
  (b) every group reaches the same total, split.barriers, after padding (the
      groups run in phase: every step of any group has one workgroup
      barrier), and the groups' tile ranges tile [0, n_tiles) in order;
  (c) every K / V stage is read only after the DMA that filled it was waited
      for (the model's waits are the kernel's vmcnt waits: all copy groups but
      the last n issued have landed) and a barrier passed, and no DMA targets
      a stage whose tile is still to be read (so every read sees the tile it
      expects). The model always takes the rare base-move fix-up at the end
      of block B, which re-reads tile jj's V stage after the step's barrier:
      that stage is free only after the next step's barrier.
"""
import os
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "cuda_fused_attention_amd", "csrc")

PROGRAM = r'''
#include "fa_fused_schedule.hpp"
#include <cstdio>
#include <vector>
using namespace fa;
constexpr int S = kFusedStages;

// A stage's state: which tile it holds, the copy group that filled it (issue
// order), and whether and when (barrier epoch) the wave has waited for it.
struct Stage { int tile = -1; int group = -1; bool landed = false; int landed_epoch = -1; };

long bad = 0;
int epoch = 0;      // workgroup barriers passed
int groups = 0;     // copy groups issued (one group = one tile's kIssues copies)
std::vector<Stage> ks, vs;

// Copy `tile` into stage `st`; the stage's previous tile must have been
// consumed: its last read happened in a step that already ended with a
// barrier (`consumed` = highest tile of that tensor whose reads are done).
void dma(std::vector<Stage>& arr, int st, int tile, int consumed) {
    if (arr[st].tile >= 0 && arr[st].tile > consumed) ++bad;
    arr[st] = Stage{tile, groups++, false, -1};
}
// s_waitcnt vmcnt(n * kIssues): every copy group except the last n issued
// has landed (copies complete in issue order).
void wait_allow(int n) {
    for (auto* a : {&ks, &vs})
        for (auto& s : *a)
            if (!s.landed && s.group >= 0 && s.group < groups - n) { s.landed = true; s.landed_epoch = epoch; }
}
void barrier() { ++epoch; }
// A read needs the expected tile, landed before the most recent barrier.
void read(std::vector<Stage>& arr, int st, int tile) {
    if (arr[st].tile != tile || !arr[st].landed || arr[st].landed_epoch >= epoch) ++bad;
}

int main() {
    for (int n_groups : {1, 2, 4})
    for (int n_tiles = 1; n_tiles <= 3000; ++n_tiles) {
        const FusedSplit sp = n_groups == 2 ? fused_split(n_tiles) : n_groups == 1 ? fused_single(n_tiles)
                                                                                   : fused_split_n(n_tiles, 4);
        if (sp.groups != n_groups) ++bad;
        int next = 0;
        for (int g = 0; g < kFusedMaxGroups; ++g) {
            if (g >= n_groups) { if (sp.count[g] != 0) ++bad; continue; }
            if (sp.first[g] != next || sp.count[g] > sp.count[0] || sp.count[g] < sp.count[0] - 1) ++bad;
            next += sp.count[g];
        }
        if (next != n_tiles) ++bad;
        for (int g = 0; g < n_groups; ++g) {
            const int cnt = sp.count[g];
            ks.assign(S, Stage{}); vs.assign(S, Stage{}); epoch = 0; groups = 0;
            // prologue: K_0 .. K_{S-1}, V_0 .. V_{S-2}
            for (int x = 0; x < S; ++x) dma(ks, x, x, -1);
            for (int x = 0; x < S - 1; ++x) dma(vs, x, x, -1);
            wait_allow(2 * S - 2);                       // Q and K_0 landed
            barrier();
            int barriers = 1;
            if (cnt > 0) read(ks, 0, 0);                 // S^T of tile 0
            wait_allow(0);                               // every prologue copy landed
            barrier(); ++barriers;
            if (cnt > 1) read(ks, 1 % S, 1);             // K operands of tile 1
            // A stage is free once its reads are followed by a barrier:
            // K_0 was read before the second prologue barrier; K_1 is read
            // after it and freed by step 0's barrier.
            int k_consumed = 0, k_pending = 1, v_consumed = -1, v_pending = -1;
            int steps = 0;
            fused_group_walk(cnt, [&](auto par, int jj) {
                ++steps;
                if (decltype(par)::value != jj % kFusedUnroll) ++bad;
                // block A: V operands of tile jj; copies of K tile jj+KAhead
                read(vs, jj % S, jj);
                dma(ks, (jj + kFusedKAhead) % S, jj + kFusedKAhead, k_consumed);
                // the step's one barrier: the last kFusedStepInFlight copy
                // groups may still fly; every LDS read issued so far has
                // completed
                wait_allow(kFusedStepInFlight);
                barrier(); ++barriers;
                v_consumed = v_pending;
                k_consumed = k_pending;
                // block B: K operands of tile jj+2; copies of V tile jj+VAhead
                if (jj + 2 < cnt) read(ks, (jj + 2) % S, jj + 2);
                k_pending = jj + 2;
                dma(vs, (jj + kFusedVAhead) % S, jj + kFusedVAhead, v_consumed);
                // end of block B, base-move fix-up: V operands of tile jj again
                read(vs, jj % S, jj);
                v_pending = jj;
            });
            if (steps != cnt) ++bad;
            if (barriers != fused_group_barriers(g, cnt)) ++bad;
            if (barriers > sp.barriers) ++bad;
        }
    }
    std::printf("%ld\n", bad);
    return bad != 0;
}
'''


def test_schedule_barriers_and_stages(tmp_path):
    src = tmp_path / "sched.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "sched"
    r = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout + out.stderr


def test_schedule_checker_catches_a_short_pipeline(tmp_path):
    """Planted mistakes: a K prefetch two tiles further ahead overwrites a
    stage still to be read; V copies one tile further ahead (with a fourth
    prologue V copy, so every other read still finds its tile) overwrite the
    stage the base-move fix-up re-reads after the barrier; a mid-step wait
    that lets one more copy group fly, and a prologue wait that lets the last
    prologue copies fly, read a stage before its copy landed. The checker must
    report each."""
    plants = [
        [("dma(ks, (jj + kFusedKAhead) % S, jj + kFusedKAhead, k_consumed);",
          "dma(ks, (jj + kFusedKAhead + 2) % S, jj + kFusedKAhead + 2, k_consumed);")],
        [("for (int x = 0; x < S - 1; ++x) dma(vs, x, x, -1);", "for (int x = 0; x < S; ++x) dma(vs, x, x, -1);"),
         ("dma(vs, (jj + kFusedVAhead) % S, jj + kFusedVAhead, v_consumed);",
          "dma(vs, (jj + kFusedVAhead + 1) % S, jj + kFusedVAhead + 1, v_consumed);")],
        [("wait_allow(kFusedStepInFlight);", "wait_allow(kFusedStepInFlight + 1);")],
        [("wait_allow(0);                               // every", "wait_allow(3);                               // every")],
    ]
    for i, subs in enumerate(plants):
        prog = PROGRAM
        for old, new in subs:
            assert old in prog
            prog = prog.replace(old, new)
        src = tmp_path / f"sched_bad{i}.cpp"
        src.write_text(prog)
        exe = tmp_path / f"sched_bad{i}"
        r = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], capture_output=True,
                           text=True)
        assert r.returncode == 0, r.stderr
        out = subprocess.run([str(exe)], capture_output=True, text=True)
        assert out.returncode != 0 and out.stdout.strip() != "0", (i, out.stdout)



LIST_PROGRAM = r'''
#include "fa_fused_schedule.hpp"
#include <cstdio>
#include <set>
using namespace fa;

int main() {
    long bad = 0;
    const int G = 4, W = 2;
    for (int e = 0; e <= 160; ++e)
    for (int l = 0; l <= 160; ++l) {
        if (e + l == 0) continue;
        const FusedSplit s = fused_split_n(e + l, G);
        const FusedListHolders h = fused_list_holders(s, e);
        // holders are exactly the groups whose items meet the half block
        auto covers = [&](int g, int half) {
            const int lo = s.first[g], hi = s.first[g] + s.count[g];
            return s.count[g] > 0 && (half == 0 ? lo < e : hi > e);
        };
        int crossing = 0;
        for (int g = 0; g < G; ++g) {
            const bool a = covers(g, 0), b = covers(g, 1);
            if (a != (g <= h.a_hi)) ++bad;
            if (b != (g >= h.b_lo && g <= h.b_hi)) ++bad;
            if (a && b) { ++crossing; if (h.cross != g) ++bad; }
        }
        if (crossing > 1 || (crossing == 0 && h.cross != G)) ++bad;
        if ((e > 0) != (h.a_hi >= 0) || (l > 0) != (h.b_hi >= 0)) ++bad;
        // finalisers: holders of the half block; one each dim half; a lone
        // holder takes both; no group finalises both half blocks
        std::set<int> fin[2];
        for (int half = 0; half < 2; ++half) {
            const int lo = half == 0 ? 0 : h.b_lo, hi = half == 0 ? h.a_hi : h.b_hi;
            if (hi < 0) continue;
            for (int dh = 0; dh < 2; ++dh) {
                const int f = fused_list_finaliser(h, half, dh);
                if (f < lo || f > hi) ++bad;
                fin[half].insert(f);
            }
            if ((lo == hi) != (fin[half].size() == 1)) ++bad;
        }
        for (int f : fin[0]) if (fin[1].count(f)) ++bad;
        // records: distinct and inside the W * (G + 1) reserved
        std::set<int> rec;
        for (int g = 0; g < G; ++g)
            for (int half = 0; half < 2; ++half) {
                if (!covers(g, half)) continue;
                for (int w = 0; w < W; ++w) {
                    const int r = fused_list_record(h, g, half, w, W);
                    if (r < 0 || r >= W * (G + 1) || !rec.insert(r).second) ++bad;
                }
            }
    }
    std::printf("%ld\n", bad);
    return bad != 0;
}
'''


def _run_list_program(tmp_path, prog, tag):
    src = tmp_path / f"list_{tag}.cpp"
    src.write_text(prog)
    exe = tmp_path / f"list_{tag}"
    r = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    return subprocess.run([str(exe)], capture_output=True, text=True)


def test_list_layout_merge_bookkeeping(tmp_path):
    """The list layout's merge plan (csrc/fa_fused_schedule.hpp, used by the
    kernel), for every pair of half-block tile counts up to 160 with four
    groups: the holders of each half block are exactly the groups whose items
    meet it, at most one group holds both, every dim half has one finaliser
    among the holders (a lone holder takes both), no group finalises both half
    blocks, and the records of all partials are distinct and within the
    reserved count."""
    out = _run_list_program(tmp_path, LIST_PROGRAM, "ok")
    assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout + out.stderr


def test_list_bookkeeping_checker_catches_mistakes(tmp_path):
    """Planted in the checked header's use: numbering records without the
    crossing group's extra slot collides records; B finalised by its first two
    holders lets a crossing group finalise both half blocks."""
    plants = [("const int r = fused_list_record(h, g, half, w, W);",
               "const int r = (g + (half == 1 && g == h.cross ? 1 : 0)) * W + w;"),
              ("const int f = fused_list_finaliser(h, half, dh);",
               "const int f = half == 0 ? fused_list_finaliser(h, half, dh) : (lo == hi ? hi : lo + dh);")]
    for i, (old, new) in enumerate(plants):
        assert old in LIST_PROGRAM
        out = _run_list_program(tmp_path, LIST_PROGRAM.replace(old, new), f"bad{i}")
        assert out.returncode != 0 and out.stdout.strip() != "0", (i, out.stdout)
