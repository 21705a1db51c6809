// Fused BF16 attention forward on gfx950 (CDNA4) MFMA — the kernel behind the
// reference's tensor-core v3 slot (kernels/v3/v3_tensorcore.cu:419-678 computes
// the same function: QK^T -> scale/mask -> online softmax -> bf16 P -> PV ->
// normalise -> bf16 O, fp32 accumulation throughout).
//
// Work layout (CDNA4-first, not a translation of the m16n8k16 design):
//
//   * A workgroup owns 32*kWpg query rows and runs two wave groups of kWpg
//     wave64s each. Wave w of group 0 and wave w of group 1 own the same 32
//     rows; group 0 walks the first half of the KV tiles, group 1 the second
//     half (split-KV inside the workgroup); their partial (max, sum, O) are
//     merged through LDS at the end. With kWpg = 4 that is two waves per SIMD.
//   * The groups ping-pong: phases alternate between an MFMA phase (PV of
//     tile k-1, then S^T of tile k) and a VALU phase (online softmax of tile
//     k), and group 1 runs one phase behind group 0. So while one wave of a
//     SIMD feeds the matrix core the other runs exp/max/convert on the VALU.
//     Every phase ends with a workgroup barrier; both groups execute the same
//     number of barriers (fa_fused_schedule.hpp).
//   * Both GEMMs use v_mfma_f32_32x32x16_bf16. QK^T is computed transposed,
//     S^T = K . Q^T (K tile from LDS = A operand, the wave's Q rows in
//     registers = B operand): lane l then holds query l % 32 and keys
//     8*(r/4) + 4*(l/32) + r%4, so a row's max and sum need one cross-lane
//     step. PV is computed as O^T = V^T . P^T: the exponentiated scores already
//     are the B operand, P never leaves registers, and O^T's layout again
//     gives lane l query l % 32, so the online-softmax rescale is per lane.
//     The A operand (8 keys of one head dim per lane) comes from the
//     row-major V tile through two ds_read_b64_tr_b16: within each group of
//     16 lanes, output lane j element r is element j%4 of the 8-byte chunk
//     addressed by source lane 4r + j/4.
//   * K and V tiles (64 keys) are copied HBM -> LDS directly with
//     global_load_lds_dwordx4 (lane l of an issue lands at base + 16*l), two
//     stages per tensor per group, issued two phases before use. The LDS rows
//     are row-major with the 16-byte chunk index XOR-swizzled per row so that
//     every ds_read_b128 (K) and ds_read_b64_tr_b16 (V) phase hits 64 distinct
//     banks; the swizzle is realised by choosing which global chunk each lane
//     fetches. Rows past the sequence end are fetched from the last valid row
//     (finite data) and masked.
//   * Scores stay in the log2 domain (scale*log2(e) folded into one FMA before
//     v_exp_f32). The exponent base (running max) is only raised when a row's
//     max grows by more than 2^8, then O and the row sum are rescaled; P stays
//     <= 256. Row sums accumulate the bf16-rounded P with v_dot2_f32_bf16, the
//     same weights the PV MFMA uses.
//   * Causal: a wave skips tiles wholly above its diagonal, only tiles that
//     cross the diagonal or the sequence end pay for the per-element mask
//     (-inf), and workgroups are issued heaviest-first. Workgroup ids are
//     remapped so that all query blocks of a (batch, head) slab run on one XCD
//     and share its L2 (measured: K and V are read from HBM once).

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <type_traits>

#include "fa_common.hpp"
#include "fa_fused_schedule.hpp"
#include "../../include/fa_mi355x.h"

namespace {

using fa::bf16x8;
using fa::f32x16;

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kTileKV = fa::kFusedTileKV;  // keys per LDS tile
constexpr float kRescaleLog2 = 8.0f;       // raise the exponent base when a row max grows by > 2^8

template <int D, int kWpg>
struct Cfg
{
    static constexpr int kRows = 32 * kWpg;               // query rows per workgroup
    static constexpr int kThreads = 128 * kWpg;           // two groups of kWpg waves
    static constexpr int kChunks = D / 8;                 // 16-byte chunks per row
    static constexpr int kTileElems = kTileKV * D;        // bf16 per K or V tile
    static constexpr int kIssues = kTileKV * kChunks / (64 * kWpg);  // DMA issues per wave per tile
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static_assert(kIssues * 64 * kWpg == kTileKV * kChunks, "tile splits evenly over a group");
    static_assert(2 * kIssues < 64, "vmcnt range");
    // the merge stages one wave's O^T (fp32) in one tile-sized LDS array
    static_assert((D / 32) * 16 * 64 * 4 == kTileElems * 2, "O^T of a wave fills one tile array");
    static_assert(kWpg <= 4, "merge staging uses four arrays");
};

// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (expcnt untouched).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that is also a compiler memory barrier (no LDS access may
// move across it). Callers wait for their own outstanding memory first.
__device__ __forceinline__ void barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 16-byte-chunk XOR swizzles (bank-conflict-free on gfx950's 64 x 4-byte banks).
// K rows are read by ds_read_b128 with 16 consecutive rows per phase.
template <int D>
__device__ __forceinline__ int swz_k(int row)
{
    return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
// V rows are read by ds_read_b64_tr_b16: 4 consecutive rows x 2 chunks per
// 16-lane group, 32 lanes per phase.
template <int D>
__device__ __forceinline__ int swz_v(int row)
{
    return D == 128 ? (2 * (row & 3) + 8 * (row & 1)) : (2 * (row & 3));
}

// One 16-byte-per-lane HBM -> LDS copy: lane l's 16 bytes from
// sbase + voff land at LDS byte address lds + 16*l (global_load_lds_dwordx4).
// Issued through inline asm so the compiler's LDS-DMA alias tracking, which
// cannot tell the pipeline stages apart, adds no waits of its own: every
// consumer of the data waits on vmcnt explicitly before a barrier. M0 needs
// one wait state between its write and the load.
__device__ __forceinline__ void dma16(const char* sbase, uint32_t voff, uint32_t lds)
{
    // Both scalar operands are uniform by construction; readfirstlane makes
    // that explicit so they are always allocated to SGPRs.
    // readfirstlane returns int: each half goes back through uint32_t before
    // widening, or a low word with bit 31 set would sign-extend into the
    // high word.
    const uint64_t base_bits = reinterpret_cast<uint64_t>(sbase);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(base_bits))));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(base_bits >> 32)));
    sbase = reinterpret_cast<const char*>((static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo));
    lds = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lds)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p)
{
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)(p)));
}

// Issue this wave's share of one K or V tile (kIssues copies of 64 x 16 B):
// block u*kWpg + wg covers rows [block*kRowsPerBlock, +kRowsPerBlock) of the
// tile. The row and tile offsets go into the uniform scalar base; the
// per-lane offset only holds the row within the block and the swizzled
// chunk. Rows past the sequence end (tail tile) are clamped to the last row.
template <int D, int kWpg, bool kIsV>
__device__ __forceinline__ void dma_tile(const uint16_t* __restrict__ slab, int kv0, int n, uint32_t stage_lds, int wg_s,
                                         int lane)
{
    using C = Cfg<D, kWpg>;
    constexpr int kRowsPerBlock = 64 / C::kChunks;
    const int sub_row = lane / C::kChunks;
    const int pchunk = lane % C::kChunks;
    if (kv0 + kTileKV <= n)
    {
#pragma unroll
        for (int u = 0; u < C::kIssues; ++u)
        {
            const int block = u * kWpg + wg_s;
            const int row0 = block * kRowsPerBlock;
            const int lchunk = pchunk ^ (kIsV ? swz_v<D>(row0 + sub_row) : swz_k<D>(row0 + sub_row));
            const char* sbase = reinterpret_cast<const char*>(slab) + static_cast<size_t>(kv0 + row0) * (D * 2);
            dma16(sbase, static_cast<uint32_t>(sub_row * (D * 2) + lchunk * 16), stage_lds + block * 1024);
        }
    }
    else
    {
#pragma unroll
        for (int u = 0; u < C::kIssues; ++u)
        {
            const int block = u * kWpg + wg_s;
            const int row = block * kRowsPerBlock + sub_row;
            const int lchunk = pchunk ^ (kIsV ? swz_v<D>(row) : swz_k<D>(row));
            const int key = min(kv0 + row, n - 1);
            dma16(reinterpret_cast<const char*>(slab), static_cast<uint32_t>(key * (D * 2) + lchunk * 16),
                  stage_lds + block * 1024);
        }
    }
}

template <int D>
struct Frag
{
    bf16x8 q[D / 16];       // Q rows (B operand of S^T), whole kernel
    f32x16 o[D / 32];       // O^T accumulators
    int k_off[D / 16];      // per-lane LDS element offsets of the K A-operand reads
    int v_off[D / 32];      // per-lane LDS element offsets of the V tr16 reads
};

// Scheduling-group masks for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// S^T (64 keys x 32 queries) = K tile . Q^T. Two operand reads run ahead of
// the MFMA stream, then each MFMA is followed by the next read, which keeps
// only a few operand registers in flight.
template <int D>
__device__ __forceinline__ void qk_tile(const uint16_t* k_stage, const Frag<D>& f, f32x16 (&s)[2])
{
#pragma unroll
    for (int b = 0; b < 2; ++b)
    {
        s[b] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
        {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(k_stage + f.k_off[ks] + b * 32 * D);
            s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, f.q[ks], s[b], 0, 0, 0);
        }
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
    for (int j = 0; j < D / 8 - 2; ++j)
    {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
}

// O^T += V^T . P^T for one tile (two tr16 reads per MFMA, kept two MFMAs
// ahead).
template <int D>
__device__ __forceinline__ void pv_tile(const uint16_t* v_stage, Frag<D>& f, const bf16x8 (&p)[4])
{
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int m = 0; m < 4; ++m)
        {
            const uint16_t* base = v_stage + f.v_off[db] + m * 16 * D;
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 8 * D));
            const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            f.o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p[m], f.o[db], 0, 0, 0);
        }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
    for (int j = 0; j < D / 8 - 2; ++j)
    {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
}

// Online softmax of one tile's scores: s -> P (bf16, B-operand layout),
// running max / sum updated, O rescaled when the exponent base moves.
template <int D, bool kCausal>
__device__ __forceinline__ void softmax_tile(Frag<D>& f, f32x16 (&s)[2], bf16x8 (&p)[4], float& m_run, float& l_run,
                                             int kv0, int n, int query, int h, float c_log2, bool masked)
{
    if (masked)  // one code path for both cases keeps register pressure flat
    {
        // Key of element r of block b is kv0 + 32b + 4h + c(r) with the
        // compile-time c(r) = 8*(r/4) + r%4; it is dead when c(r) >= limit_b.
        // Comparing against immediates keeps 32 key indices out of registers.
        const int first_dead = kCausal ? min(n, query + 1) : n;
#pragma unroll
        for (int b = 0; b < 2; ++b)
        {
            const int limit = first_dead - kv0 - 32 * b - 4 * h;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (8 * (r >> 2) + (r & 3) >= limit) s[b][r] = -INFINITY;
        }
    }

    // IEEE maximum (v_maximum3_f32) needs no operand canonicalisation; the
    // other half of the row sits in lane l^32 (v_permlane32_swap).
    float mx = __builtin_elementwise_maximum(s[0][0], s[1][0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(s[0][r], s[1][r]));
    {
        const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
        const auto swapped = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
        mx = __builtin_elementwise_maximum(__builtin_bit_cast(float, swapped[0]), __builtin_bit_cast(float, swapped[1]));
    }
    mx *= c_log2;

    if (__any(mx > m_run + kRescaleLog2))
    {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) f.o[db][r] *= alpha;
    }
    const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;

#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            p[m][e] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[m >> 1][8 * (m & 1) + e], c_log2, -m_use)));

    const fa::bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int e = 0; e < 8; e += 2)
        {
            const fa::bf16x2 pair = {p[m][e], p[m][e + 1]};
            l_run = __builtin_amdgcn_fdot2_f32_bf16(pair, ones, l_run, false);
        }
}

template <int D, int kWpg, bool kCausal>
__global__ __launch_bounds__(128 * kWpg) void fused_attention_kernel(const uint16_t* __restrict__ q,
                                                                     const uint16_t* __restrict__ k,
                                                                     const uint16_t* __restrict__ v,
                                                                     uint16_t* __restrict__ o, int n,
                                                                     int q_blocks, int total_blocks,
                                                                     float c_log2)
{
    using C = Cfg<D, kWpg>;
    // Per group: two K stages and two V stages at compile-time offsets of one
    // LDS array, so every operand read is a per-lane base plus an immediate.
    __shared__ __attribute__((aligned(16))) uint16_t lds[8 * C::kTileElems];
    uint16_t* const k00 = lds + 0 * C::kTileElems;
    uint16_t* const k01 = lds + 1 * C::kTileElems;
    uint16_t* const v00 = lds + 2 * C::kTileElems;
    uint16_t* const v01 = lds + 3 * C::kTileElems;
    uint16_t* const k10 = lds + 4 * C::kTileElems;
    uint16_t* const k11 = lds + 5 * C::kTileElems;
    uint16_t* const v10 = lds + 6 * C::kTileElems;
    uint16_t* const v11 = lds + 7 * C::kTileElems;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = wave / kWpg;      // KV half
    const int wg = wave % kWpg;       // row block within the workgroup
    const int wg_s = __builtin_amdgcn_readfirstlane(wg);  // same value, in an SGPR
    const int i = lane & 31;
    const int h = lane >> 5;

    const int logical = fa::xcd_remap(static_cast<int>(blockIdx.x), total_blocks);
    const int slab = logical / q_blocks;
    const int qb_in = logical % q_blocks;
    const int qb = kCausal ? (q_blocks - 1 - qb_in) : qb_in;  // causal: heaviest first
    const int q0 = qb * C::kRows;
    const int wq0 = q0 + 32 * wg;

    const size_t slab_off = static_cast<size_t>(slab) * n * D;
    const uint16_t* q_slab = q + slab_off;
    const uint16_t* k_slab = k + slab_off;
    const uint16_t* v_slab = v + slab_off;

    const int last_key = kCausal ? min(q0 + C::kRows - 1, n - 1) : n - 1;
    const int n_tiles = last_key / kTileKV + 1;
    const fa::FusedSplit split = fa::fused_split(n_tiles);

    // Tiles from t_mask on need the per-element mask (sequence tail, or this
    // wave's diagonal); tiles after t_last lie wholly above the diagonal.
    const int t_tail = (n % kTileKV) ? n / kTileKV : n_tiles;
    const int t_diag = kCausal ? (wq0 + 1) / kTileKV : n_tiles;
    const int t_mask = min(t_tail, t_diag);
    // Dense: t_last is n_tiles - 1, passed through readfirstlane so the
    // compiler cannot fold the per-phase tests away; folded, it merges the
    // phases' blocks and its hoisting then spills at head_dim 128.
    const int t_last = kCausal ? min((wq0 + 31) / kTileKV, n_tiles - 1) : __builtin_amdgcn_readfirstlane(n_tiles - 1);

    Frag<D> f;
    const int query = wq0 + i;
    float m_run = -INFINITY;
    float l_run = 0.0f;

    auto run_group = [&](auto gtag) {
        constexpr int G = decltype(gtag)::value;
        uint16_t* const kb0 = G == 0 ? k00 : k10;
        uint16_t* const kb1 = G == 0 ? k01 : k11;
        uint16_t* const vb0 = G == 0 ? v00 : v10;
        uint16_t* const vb1 = G == 0 ? v01 : v11;
        const int tb = G == 0 ? 0 : split.first1;        // first tile of this group
        const int cnt = G == 0 ? split.count0 : split.count1;

        // Every DMA issue point copies a fixed number of tiles so the vmcnt
        // waits below are constants. A tile index past the end is clamped
        // to the last tile; such a copy lands in a stage nobody reads again.
        auto kv_at = [&](int tile) { return min(tile, n_tiles - 1) * kTileKV; };

        // Prologue DMAs: V_0, K_0, K_1 of this group.
        dma_tile<D, kWpg, true>(v_slab, kv_at(tb), n, lds_addr(vb0), wg_s, lane);
        dma_tile<D, kWpg, false>(k_slab, kv_at(tb), n, lds_addr(kb0), wg_s, lane);
        dma_tile<D, kWpg, false>(k_slab, kv_at(tb + 1), n, lds_addr(kb1), wg_s, lane);

#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
        {
            if (query < n)
                f.q[ks] = *reinterpret_cast<const bf16x8*>(q_slab + static_cast<size_t>(query) * D + 16 * ks + 8 * h);
            else
                f.q[ks] = bf16x8{};
        }
#pragma unroll
        for (int db = 0; db < D / 32; ++db) f.o[db] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) f.k_off[ks] = i * D + (((2 * ks + h) ^ swz_k<D>(i)) << 3);
        {
            // V tr16 source-lane role: group g16 = lane/16 -> (h = g16/2, dim
            // half g16%2); s16 = lane%16 -> row s16/4 of a 4-row group, 4-dim
            // piece s16%4.
            const int g16 = lane >> 4;
            const int s16 = lane & 15;
            const int vr = 4 * (g16 >> 1) + (s16 >> 2);
            const int dim = 16 * (g16 & 1) + 4 * (s16 & 3);
#pragma unroll
            for (int db = 0; db < D / 32; ++db)
            {
                const int col = 32 * db + dim;
                f.v_off[db] = vr * D + (((col >> 3) ^ swz_v<D>(vr)) << 3) + (col & 7);
            }
        }

        wait_vm_lgkm0<0>();
        barrier();                          // prologue tiles resident
        if (G == 1) barrier();              // group 1 runs one phase behind

        f32x16 s[2];
        bf16x8 p[4];

        // MFMA phase of local step kk: PV of tile kk-1 (V stage (kk-1)%2),
        // then S^T of tile kk (K stage kk%2).
        auto mfma_phase = [&](auto par_tag, int kk) {
            constexpr int kPar = decltype(par_tag)::value;   // kk % 2
            const int t_prev = tb + kk - 1;
            if (kk >= 1 && t_prev <= t_last) pv_tile<D>(kPar ? vb0 : vb1, f, p);
            if (kk < cnt && tb + kk <= t_last) qk_tile<D>(kPar ? kb1 : kb0, f, s);
            wait_vm_lgkm0<63>();
            barrier();
        };
        // VALU phase of local step kk: refill V stage (kk+1)%2 and K stage
        // kk%2, softmax of tile kk, then wait for the previous step's DMAs.
        auto valu_phase = [&](auto par_tag, int kk) {
            constexpr int kPar = decltype(par_tag)::value;
            const int t = tb + kk;
            dma_tile<D, kWpg, true>(v_slab, kv_at(t + 1), n, lds_addr(kPar ? vb0 : vb1), wg_s, lane);
            dma_tile<D, kWpg, false>(k_slab, kv_at(t + 2), n, lds_addr(kPar ? kb1 : kb0), wg_s, lane);
            if (t <= t_last)
                softmax_tile<D, kCausal>(f, s, p, m_run, l_run, t * kTileKV, n, query, h, c_log2, t >= t_mask);
            // Everything but this step's DMAs must have landed.
            wait_vm_lgkm0<2 * C::kIssues>();
            barrier();
        };

        fa::fused_group_walk(cnt, mfma_phase, valu_phase);
        // Pad to the common barrier count of both groups.
        for (int b = fa::fused_group_barriers(G, cnt); b < split.barriers; ++b) barrier();
        // Drain this wave's last (unused) copies before LDS is reused below.
        wait_vm_lgkm0<0>();
        barrier();
    };

    if (grp == 0) run_group(std::integral_constant<int, 0>{});
    else run_group(std::integral_constant<int, 1>{});

    // Merge: group 1 stages its (exponent base, partial sums, O^T) in LDS,
    // group 0 folds them into its own and writes O. All DMAs have landed
    // (every wave drained its own before the last barrier).
    float* const ostage = reinterpret_cast<float*>(wg == 0 ? k10 : wg == 1 ? k11 : wg == 2 ? v10 : v11);
    float* const ml_stage = reinterpret_cast<float*>(k00);
    if (grp == 1)
    {
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) ostage[(db * 16 + r) * 64 + lane] = f.o[db][r];
        ml_stage[wg * 128 + lane] = m_run;
        ml_stage[wg * 128 + 64 + lane] = l_run;
    }
    wait_vm_lgkm0<0>();
    barrier();
    if (grp == 1) return;

    {
        const float m1 = ml_stage[wg * 128 + lane];
        const float l1 = ml_stage[wg * 128 + 64 + lane];
        const float m = fmaxf(m_run, m1);
        const float a0 = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
        const float a1 = (m1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
        l_run = l_run * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) f.o[db][r] = f.o[db][r] * a0 + ostage[(db * 16 + r) * 64 + lane] * a1;
    }

    // Epilogue: the two lane halves hold partial row sums of the same query.
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (query < n)
    {
        uint16_t* o_row = o + slab_off + static_cast<size_t>(query) * D;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g)
            {
                uint2 packed;
                packed.x = fa::pack_bf16x2(f.o[db][4 * g + 0] * inv, f.o[db][4 * g + 1] * inv);
                packed.y = fa::pack_bf16x2(f.o[db][4 * g + 2] * inv, f.o[db][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(o_row + 32 * db + 8 * g + 4 * h) = packed;
            }
    }
}

template <int D, int kWpg, bool kCausal>
const void* kernel_ptr()
{
    return reinterpret_cast<const void*>(&fused_attention_kernel<D, kWpg, kCausal>);
}

template <int kWpg>
const void* pick_kernel(int head_dim, bool causal)
{
    if (head_dim == 64) return causal ? kernel_ptr<64, kWpg, true>() : kernel_ptr<64, kWpg, false>();
    if (head_dim == 128) return causal ? kernel_ptr<128, kWpg, true>() : kernel_ptr<128, kWpg, false>();
    return nullptr;
}

template <int D, int kWpg, bool kCausal>
void launch_typed(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int n, int q_blocks,
                  int total, float c_log2, hipStream_t stream)
{
    hipLaunchKernelGGL((fused_attention_kernel<D, kWpg, kCausal>), dim3(static_cast<unsigned>(total)),
                       dim3(Cfg<D, kWpg>::kThreads), 0, stream, q, k, v, o, n, q_blocks, total, c_log2);
}

template <int kWpg>
int launch_fused(const void* q, const void* k, const void* v, void* o, int batch, int heads, int seq_len,
                 int head_dim, int causal, void* stream_ptr)
{
    if (head_dim != 64 && head_dim != 128) return FA_ERROR_UNSUPPORTED;
    if (batch < 0 || heads < 0 || seq_len < 0) return hipErrorInvalidValue;
    const long long bh = static_cast<long long>(batch) * heads;
    if (bh == 0 || seq_len == 0) return hipSuccess;
    if (!q || !k || !v || !o) return hipErrorInvalidValue;
    // 16-byte vector / LDS-DMA loads and 8-byte stores need aligned bases.
    const uintptr_t mis = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
    if (mis & 15u) return hipErrorInvalidValue;
    // DMA offsets are 32-bit byte offsets within one (batch, head) slab.
    if (static_cast<long long>(seq_len) * head_dim * 2 > 0x7fffffffLL) return hipErrorInvalidValue;
    constexpr int rows = 32 * kWpg;
    const long long q_blocks = (static_cast<long long>(seq_len) + rows - 1) / rows;
    const long long total = bh * q_blocks;
    if (total > 0x7fffffffLL / (128 * kWpg)) return hipErrorInvalidValue;

    const float c_log2 = fa_default_scale(head_dim) * fa::kLog2e;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const auto* qb = static_cast<const uint16_t*>(q);
    const auto* kb = static_cast<const uint16_t*>(k);
    const auto* vb = static_cast<const uint16_t*>(v);
    auto* ob = static_cast<uint16_t*>(o);
    const int qbk = static_cast<int>(q_blocks);
    const int tot = static_cast<int>(total);
    if (head_dim == 64)
    {
        if (causal) launch_typed<64, kWpg, true>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
        else launch_typed<64, kWpg, false>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
    }
    else
    {
        if (causal) launch_typed<128, kWpg, true>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
        else launch_typed<128, kWpg, false>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
    }
    return static_cast<int>(hipGetLastError());
}

template <int kWpg>
int query_fused(int head_dim, fa_tiling_info* info)
{
    if (!info) return hipErrorInvalidValue;
    *info = fa_tiling_info{};
    if (head_dim != 64 && head_dim != 128) return hipSuccess;  // supported = 0
    info->supported = 1;
    info->block_size = 128 * kWpg;
    info->waves_per_block = 2 * kWpg;
    info->tile_kv = kTileKV;
    info->rows_per_block = 32 * kWpg;

    const void* func = pick_kernel<kWpg>(head_dim, false);
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, func);
    if (e != hipSuccess) return e;
    info->shared_bytes_per_block = static_cast<int>(attr.sharedSizeBytes);
    info->registers_per_thread = attr.numRegs;
    info->local_bytes_per_thread = static_cast<int>(attr.localSizeBytes);

    int blocks = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, func, 128 * kWpg, 0);
    if (e != hipSuccess) return e;
    info->max_blocks_per_sm = blocks;

    int device = 0;
    if ((e = hipGetDevice(&device)) != hipSuccess) return e;
    int lds_per_cu = 0;
    if ((e = hipDeviceGetAttribute(&lds_per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device)) !=
        hipSuccess)
        return e;
    info->device_shared_bytes_per_sm = lds_per_cu;
    info->shared_limited_blocks_per_sm =
        info->shared_bytes_per_block > 0 ? lds_per_cu / info->shared_bytes_per_block : 0;
    int cus = 0;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess) return e;
    info->compute_units = cus;
    // hipFuncAttributes reports one register count (numRegs); AGPR use is
    // visible in the compiler's resource remarks, not through this API.
    info->agprs_per_thread = 0;
    return hipSuccess;
}

// kernels/v3/v3_tensorcore.cu:795-818 accounting for this tiling: Q read and
// O written once, K and V tiles counted once per query block that loads them.
double blocked_hbm_bytes(int batch, int heads, int seq_len, int head_dim, int causal, int rows_per_block)
{
    if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0.0;
    const double element = 2.0;
    const double slabs = static_cast<double>(batch) * heads;
    const int row_blocks = (seq_len + rows_per_block - 1) / rows_per_block;
    double bytes = 2.0 * slabs * seq_len * static_cast<double>(head_dim) * element;
    double kv_tiles = 0.0;
    for (int block = 0; block < row_blocks; ++block)
    {
        const int q_max = block * rows_per_block + rows_per_block - 1;
        const int key_limit = causal ? (q_max < seq_len - 1 ? q_max : seq_len - 1) : seq_len - 1;
        kv_tiles += static_cast<double>(key_limit / kTileKV + 1);
    }
    bytes += 2.0 * slabs * kv_tiles * kTileKV * head_dim * element;
    return bytes;
}

}  // namespace

extern "C" {

int fa_tensorcore_v3_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

int fa_launch_attention_tensorcore_v3(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                                      int seq_len, int head_dim, int causal, void* stream)
{
    return launch_fused<4>(q, k, v, o, batch, heads, seq_len, head_dim, causal, stream);
}

int fa_query_tensorcore_v3(int head_dim, fa_tiling_info* info) { return query_fused<4>(head_dim, info); }

double fa_tensorcore_v3_hbm_bytes(int batch, int heads, int seq_len, int head_dim, int causal)
{
    return blocked_hbm_bytes(batch, heads, seq_len, head_dim, causal, 128);
}

int fa_tensorcore_v3b_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

int fa_launch_attention_tensorcore_v3b(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                                       int seq_len, int head_dim, int causal, void* stream)
{
    return launch_fused<2>(q, k, v, o, batch, heads, seq_len, head_dim, causal, stream);
}

int fa_query_tensorcore_v3b(int head_dim, fa_tiling_info* info) { return query_fused<2>(head_dim, info); }

double fa_tensorcore_v3b_hbm_bytes(int batch, int heads, int seq_len, int head_dim, int causal)
{
    return blocked_hbm_bytes(batch, heads, seq_len, head_dim, causal, 64);
}

}  // extern "C"
