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
constexpr int kFusedStages = 4;   // LDS stages per tensor (K, V) per wave group

// Pipeline of one group, local step jj (tile jj of the group):
//   block A  read the V operands of tile jj (LDS -> registers); DMA K tile
//            jj + kFusedKAhead (its copies spread between the MFMAs);
//   barrier  wait until only the DMAs of steps jj-1 and jj are in flight and
//            every LDS read issued so far has completed; workgroup barrier;
//   block B  read the K operands of tile jj + 2; DMA V tile jj + kFusedVAhead;
//            rarely (an exponent-base move), read tile jj's V operands
//            again at the end of the block.
// One barrier per step covers both hazards: K_{jj+2} and V_{jj+1} landed
// before it (read after it), and every stage a later copy overwrites was
// last read before it or before the previous step's barrier (V_{jj-1}'s
// stage, the target of block B's copy, was last read in step jj - 1).
// The prologue copies K_0 .. K_3 and V_0 .. V_2, waits for K_0 and reads
// its operands, then waits for every prologue copy and reads K_1's operands.
constexpr int kFusedKAhead = kFusedStages;      // into K_jj's stage (read in step jj - 2)
constexpr int kFusedVAhead = kFusedStages - 1;  // into V_{jj-1}'s stage (read in step jj - 1)

struct FusedSplit
{
    int count0;    // KV tiles walked by group 0: [0, count0)
    int first1;    // first tile of group 1
    int count1;    // KV tiles walked by group 1: [first1, first1 + count1)
    int barriers;  // barriers each group executes before the merge
};

// Barriers group `g` executes for `count` tiles: one after the prologue DMAs,
// one after the prologue's first S tile, and one per step. Both groups run
// in phase, pad to FusedSplit::barriers and run the same fixed tail (drain,
// merge).
FA_HD inline int fused_group_barriers(int /*g*/, int count) { return 2 + count; }

// The step walk of one group over its `count` tiles: step(kk, jj) for
// jj = 0 .. count-1 with kk = jj % kFusedUnroll as a compile-time
// std::integral_constant: kk % kFusedStages is the LDS stage rotation and
// kk % 2 the register double buffer of S and P. Each step runs exactly one
// workgroup barrier.
constexpr int kFusedUnroll = kFusedStages;
static_assert(kFusedUnroll % 2 == 0, "the S / P double buffer needs an even unroll");

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
        ++jj;
    }
}

FA_HD inline FusedSplit fused_split(int n_tiles)
{
    FusedSplit s;
    s.count0 = (n_tiles + 1) / 2;
    s.first1 = s.count0;
    s.count1 = n_tiles - s.count0;
    const int b0 = fused_group_barriers(0, s.count0);
    const int b1 = fused_group_barriers(1, s.count1);
    s.barriers = b0 > b1 ? b0 : b1;
    return s;
}

// The same walk for a workgroup with one wave group (no split of the KV
// range): group 0 takes every tile.
FA_HD inline FusedSplit fused_single(int n_tiles)
{
    FusedSplit s;
    s.count0 = n_tiles;
    s.first1 = n_tiles;
    s.count1 = 0;
    s.barriers = fused_group_barriers(0, n_tiles);
    return s;
}

}  // namespace fa
