// Phase / barrier schedule of the fused kernel's two wave groups, shared by
// the device code and a host-side checker (tests compile this header with a
// plain C++ compiler and verify that both groups always execute the same
// number of workgroup barriers).
#pragma once

#include <type_traits>

#if defined(__HIPCC__) || defined(__HIP__)
#define FA_HD __host__ __device__
#else
#define FA_HD
#endif

namespace fa {

constexpr int kFusedTileKV = 64;

struct FusedSplit
{
    int count0;    // KV tiles walked by group 0: [0, count0)
    int first1;    // first tile of group 1
    int count1;    // KV tiles walked by group 1: [first1, first1 + count1)
    int barriers;  // barriers each group executes before the merge
};

// Barriers group `g` executes for `count` tiles: one after the prologue DMAs,
// one per MFMA phase (count + 1 of them: PV of the previous tile, S^T of the
// current) and one per VALU phase (count), plus group 1's initial idle phase.
// Both groups then pad to FusedSplit::barriers and run the same fixed tail
// (drain, merge), so only this group-dependent part needs checking.
FA_HD inline int fused_group_barriers(int g, int count)
{
    return 1 + (g == 1 ? 1 : 0) + (count + 1) + count;
}

// The phase walk of one group over its `count` tiles: MFMA phase 0, then
// (VALU phase kk, MFMA phase kk+1) for kk = 0 .. count-1. Each callback runs
// exactly one workgroup barrier; the first argument is kk % 2 as a
// compile-time std::integral_constant (the LDS stage parity).
template <class MfmaPhase, class ValuPhase>
FA_HD inline void fused_group_walk(int count, MfmaPhase&& mfma_phase, ValuPhase&& valu_phase)
{
    int kk = 0;
    for (;;)
    {
        mfma_phase(std::integral_constant<int, 0>{}, kk);
        if (kk >= count) break;
        valu_phase(std::integral_constant<int, 0>{}, kk);
        ++kk;
        mfma_phase(std::integral_constant<int, 1>{}, kk);
        if (kk >= count) break;
        valu_phase(std::integral_constant<int, 1>{}, kk);
        ++kk;
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

}  // namespace fa
