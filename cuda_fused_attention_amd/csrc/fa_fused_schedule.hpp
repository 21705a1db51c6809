// Tile / stage / barrier schedule of the fused kernel's two wave groups,
// shared by the device code and a host-side checker (tests compile this
// header with a plain C++ compiler and replay the walk: both groups must
// execute the same number of workgroup barriers, every LDS stage must be
// free when a DMA is issued into it and landed before it is read).
#pragma once

#include <type_traits>

#if defined(__HIPCC__) || defined(__HIP__)
#define FA_HD __host__ __device__
#else
#define FA_HD
#endif

namespace fa {

constexpr int kFusedTileKV = 32;  // keys per LDS tile
constexpr int kFusedStages = 3;   // LDS stages per tensor (K, V) per wave group

// Pipeline of one group, local step jj (tile jj of the group):
//   block A  read the V operands of tile jj (LDS -> registers); DMA K tile
//            jj + kFusedKAhead (its copies spread between the MFMAs);
//   barrier  wait until only the last kFusedStepInFlight copy groups are in
//            flight (block A's K copy) and every LDS read issued so far has
//            completed; workgroup barrier;
//   block B  read the K operands of tile jj + 2; DMA V tile jj + kFusedVAhead;
//            rarely (an exponent-base move), read tile jj's V operands
//            again at the end of the block.
// One barrier per step covers both hazards: K_{jj+2} (copied in block A of
// step jj-1) and V_{jj+1} (block B of step jj-1) landed before it and are
// read after it, and every stage a later copy overwrites was last read
// before it or before the previous step's barrier (V_{jj-1}'s stage, the
// target of block B's copy, was last read in step jj - 1). A copy thus has
// one to one and a half steps to land; with four stages it had two and a
// half, which measured no faster and costs a deeper prologue.
// The prologue copies K_0 .. K_{S-1} and V_0 .. V_{S-2}, waits for K_0 and
// reads its operands, then waits for every prologue copy and reads K_1's
// operands.
constexpr int kFusedKAhead = kFusedStages;      // into K_jj's stage (read in step jj - 2)
constexpr int kFusedVAhead = kFusedStages - 1;  // into V_{jj-1}'s stage (read in step jj - 1)
// Copy groups (one group = one tile's copies) still in flight at a step's
// barrier once K_{jj+2} and V_{jj+1} have landed: those issued after V_{jj+1}.
constexpr int kFusedStepInFlight = 2 * kFusedStages - 5;
static_assert(kFusedStages >= 3, "K_{jj+2} is read in the step that copies K_{jj+S}: S >= 3");

constexpr int kFusedMaxGroups = 4;  // wave groups (KV streams) per workgroup: 1, 2 or 4

struct FusedSplit
{
    int groups;                  // wave groups sharing the KV range
    int first[kFusedMaxGroups];  // first tile walked by group g
    int count[kFusedMaxGroups];  // KV tiles walked by group g: [first[g], first[g] + count[g])
    int barriers;                // barriers each group executes before the merge
};

// Barriers group `g` executes for `count` tiles: one after the prologue DMAs,
// one after the prologue's first S tile, and one per step. Both groups run
// in phase, pad to FusedSplit::barriers and run the same fixed tail (drain,
// merge).
FA_HD inline int fused_group_barriers(int /*g*/, int count) { return 2 + count; }

// The step walk of one group over its `count` tiles: step(kk, jj) for
// jj = 0 .. count-1 with kk = jj % kFusedUnroll as a compile-time
// std::integral_constant: kk % kFusedStages is the LDS stage rotation and
// kk % 2 the register double buffer of S and P (kFusedUnroll is the least
// common multiple of the two). Each step runs exactly one workgroup barrier.
constexpr int kFusedUnroll = kFusedStages % 2 == 0 ? kFusedStages : 2 * kFusedStages;
static_assert(kFusedUnroll % 2 == 0 && kFusedUnroll % kFusedStages == 0, "stage rotation and double buffer");

static_assert(kFusedUnroll == 6, "fused_group_walk is written out for six steps per pass");

// Written out step by step: a recursive template form of the same walk
// made the compiler keep 10-16 more VGPRs live in the kernel.
template <class Step>
FA_HD inline void fused_group_walk(int count, Step&& step)
{
    int jj = 0;
    while (jj < count)
    {
        step(std::integral_constant<int, 0>{}, jj);
        if (++jj >= count) break;
        step(std::integral_constant<int, 1>{}, jj);
        if (++jj >= count) break;
        step(std::integral_constant<int, 2>{}, jj);
        if (++jj >= count) break;
        step(std::integral_constant<int, 3>{}, jj);
        if (++jj >= count) break;
        step(std::integral_constant<int, 4>{}, jj);
        if (++jj >= count) break;
        step(std::integral_constant<int, 5>{}, jj);
        ++jj;
    }
}

// The KV range of n_tiles tiles split over `groups` wave groups in order:
// contiguous ranges, the earlier groups one tile longer when the count does
// not divide evenly. Every group pads to the longest group's barrier count.
FA_HD inline FusedSplit fused_split_n(int n_tiles, int groups)
{
    FusedSplit s;
    s.groups = groups;
    const int base = n_tiles / groups;
    const int rem = n_tiles % groups;
    int first = 0;
    for (int g = 0; g < kFusedMaxGroups; ++g)
    {
        s.count[g] = g < groups ? base + (g < rem ? 1 : 0) : 0;
        s.first[g] = first;
        first += s.count[g];
    }
    s.barriers = fused_group_barriers(0, s.count[0]);
    return s;
}

// Two groups: group 0 walks the first half of the KV tiles, group 1 the rest.
FA_HD inline FusedSplit fused_split(int n_tiles) { return fused_split_n(n_tiles, 2); }

// One wave group (no split of the KV range): group 0 takes every tile.
FA_HD inline FusedSplit fused_single(int n_tiles) { return fused_split_n(n_tiles, 1); }

// The list layout's merge bookkeeping. The workgroup's work list is the K/V
// tiles of half block A (items [0, e_items)) followed by those of half block
// B; the split gives each group a contiguous range of items. The holders of
// a half block are the groups whose range covers some of its items: A's are
// [0, a_hi], B's [b_lo, b_hi]; at most one group (cross) covers both, and it
// then holds two partials. Each head-dim half dh of a half block's rows is
// finalised by one holder: a lone holder takes both halves, otherwise groups
// 0 and 1 finalise A and the last two holders B, so no group finalises both
// half blocks (whenever a group crosses, every group has items and B's last
// holder is the last group).
struct FusedListHolders
{
    int cross;  // the group holding partials of both half blocks, or groups
    int a_hi;   // A's holders are groups [0, a_hi] (-1: none)
    int b_lo;   // B's holders are groups [b_lo, b_hi] (b_hi -1: none)
    int b_hi;
};

FA_HD inline FusedListHolders fused_list_holders(const FusedSplit& s, int e_items)
{
    FusedListHolders r{s.groups, -1, s.groups, -1};
    for (int g = 0; g < s.groups; ++g)
    {
        const int g0 = s.first[g];
        const int gc = s.count[g];
        if (gc > 0 && g0 < e_items) r.a_hi = g;
        if (gc > 0 && g0 + gc > e_items)
        {
            if (r.b_lo > g) r.b_lo = g;
            r.b_hi = g;
        }
        if (g0 < e_items && e_items < g0 + gc) r.cross = g;
    }
    return r;
}

// Finaliser of head-dim half dh of half block `half` (0: A, 1: B).
FA_HD inline int fused_list_finaliser(const FusedListHolders& h, int half, int dh)
{
    if (half == 0) return h.a_hi == 0 ? 0 : dh;
    return h.b_hi == h.b_lo ? h.b_hi : h.b_hi - 1 + dh;
}

// Merge record of group g's partial of half block `half` for the wave with
// slot index w of `waves` per group: records are numbered in list order
// (the crossing group's two partials take two consecutive numbers), so at
// most waves * (groups + 1) records exist.
FA_HD inline int fused_list_record(const FusedListHolders& h, int g, int half, int w, int waves)
{
    const int part = (half == 1 && g == h.cross) ? 1 : 0;
    return (g + part + (h.cross < g ? 1 : 0)) * waves + w;
}

}  // namespace fa
