// Fused BF16 attention forward on gfx950 (CDNA4) MFMA — the kernel behind the
// reference's tensor-core v3 slot (kernels/v3/v3_tensorcore.cu:419-678 computes
// the same function: QK^T -> scale/mask -> online softmax -> bf16 P -> PV ->
// normalise -> bf16 O, fp32 accumulation throughout).
//
// Layout of the work (CDNA4-first, not a translation of the m16n8k16 design):
//
//   * One workgroup = kWaves wave64s; each wave owns 32 query rows. Both
//     GEMMs use v_mfma_f32_32x32x16_bf16 (32x32 fp32 accumulator tile, 16
//     lanes... of K-depth per instruction).
//   * QK^T is computed transposed, S^T = K . Q^T: the K tile (from LDS) is the
//     A operand and the wave's Q rows (registers, loaded once) the B operand.
//     In the 32x32 accumulator layout lane l then holds column j = l % 32 —
//     one query row — and 16 key rows i = 8*(r/4) + 4*(l/32) + r%4. A query's
//     64 scores of a KV tile sit in two lanes (l and l^32), so the online
//     softmax needs one cross-lane step per row, everything else is in-lane.
//   * PV is computed transposed too, O^T = V^T . P^T: the exponentiated scores
//     are already laid out as the B operand (query = l % 32, 8 keys per lane),
//     so P never leaves registers; the A operand is V^T, which is staged in
//     LDS transposed ([dim][key]) while being copied from HBM. The key order
//     inside each 16-key group of that LDS tile swaps bits 2 and 3 of the key
//     index, which makes the 8 keys an MFMA lane needs contiguous (one 16-byte
//     LDS read). O^T's layout again gives lane l query l % 32, so the online
//     softmax rescale is a per-lane multiply.
//   * K and V^T tiles are double buffered in LDS with an XOR swizzle of the
//     16-byte chunk index (row & 7) so 8 consecutive rows read by one LDS
//     phase hit distinct banks. The next tile is fetched into registers before
//     the current tile's MFMAs and written to the other LDS buffer after them:
//     one barrier per KV tile.
//   * Scores are kept in the log2 domain (scale * log2(e) folded into one FMA
//     before v_exp_f32); masked scores are -inf, and a row whose running max is
//     still -inf uses 0 as its exponent base, so no NaN can form.
//   * Causal: tiles above a wave's diagonal are skipped, only tiles that cross
//     the diagonal or the sequence end pay for the per-element mask, and
//     workgroups are issued heaviest-first. Workgroup ids are remapped so that
//     all query blocks of a (batch, head) slab run on one XCD and share its L2.

#include <cmath>
#include <cstdint>
#include <cstdio>

#include "fa_common.hpp"
#include "../../include/fa_mi355x.h"

namespace {

using fa::bf16x8;
using fa::f32x16;

constexpr int kTileKV = 64;  // keys per LDS tile

template <int D, int kWaves>
struct Cfg
{
    static constexpr int kRows = 32 * kWaves;               // query rows per workgroup
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kKElems = kTileKV * D;             // bf16 per K stage
    static constexpr int kVElems = D * kTileKV;             // bf16 per V^T stage
    static constexpr int kLdsElems = 2 * (kKElems + kVElems);
    static constexpr int kLdsBytes = 2 * kLdsElems;
    static constexpr int kQSteps = D / 16;                  // MFMA K-steps of S^T
    static constexpr int kDBlocks = D / 32;                 // 32-dim blocks of O^T
    static constexpr int kRowChunks = D / 8;                // 16-byte chunks per K row
    static constexpr int kKLoads = kTileKV * kRowChunks / kThreads;
    static constexpr int kVUnits = (kTileKV / 4) * kRowChunks;  // 4 keys x 8 dims each
    static constexpr int kVLoads = (kVUnits + kThreads - 1) / kThreads;
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static_assert((kTileKV * kRowChunks) % kThreads == 0, "K staging splits evenly");
};

// Element offset of the 16-byte chunk `chunk` of row `row` in a swizzled tile
// whose rows hold `row_elems` bf16.
template <int kRowElems>
__device__ __forceinline__ int swz(int row, int chunk)
{
    return row * kRowElems + ((chunk ^ (row & 7)) << 3);
}

// Position of key `key` (0..63) inside a V^T LDS row: bits 2 and 3 swapped.
__device__ __forceinline__ int vt_pos(int key)
{
    return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

template <int D, int kWaves>
struct TileRegs
{
    uint4 k[Cfg<D, kWaves>::kKLoads];
    uint4 v[Cfg<D, kWaves>::kVLoads][4];
};

template <int D, int kWaves>
__device__ __forceinline__ void load_tile(TileRegs<D, kWaves>& regs, const uint16_t* __restrict__ k_slab,
                                          const uint16_t* __restrict__ v_slab, int kv0, int n, int tid)
{
    using C = Cfg<D, kWaves>;
#pragma unroll
    for (int u = 0; u < C::kKLoads; ++u)
    {
        const int c = tid + u * C::kThreads;
        const int row = c / C::kRowChunks;
        const int chunk = c % C::kRowChunks;
        const int key = kv0 + row;
        regs.k[u] = key < n ? *reinterpret_cast<const uint4*>(k_slab + static_cast<size_t>(key) * D + chunk * 8)
                            : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < C::kVLoads; ++u)
    {
        const int unit = tid + u * C::kThreads;
        const int quad = unit / C::kRowChunks;
        const int chunk = unit % C::kRowChunks;
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int key = kv0 + quad * 4 + j;
            regs.v[u][j] = (unit < C::kVUnits && key < n)
                               ? *reinterpret_cast<const uint4*>(v_slab + static_cast<size_t>(key) * D + chunk * 8)
                               : make_uint4(0, 0, 0, 0);
        }
    }
}

template <int D, int kWaves>
__device__ __forceinline__ void store_tile(const TileRegs<D, kWaves>& regs, uint16_t* k_lds, uint16_t* vt_lds,
                                           int tid)
{
    using C = Cfg<D, kWaves>;
#pragma unroll
    for (int u = 0; u < C::kKLoads; ++u)
    {
        const int c = tid + u * C::kThreads;
        const int row = c / C::kRowChunks;
        const int chunk = c % C::kRowChunks;
        *reinterpret_cast<uint4*>(k_lds + swz<D>(row, chunk)) = regs.k[u];
    }
#pragma unroll
    for (int u = 0; u < C::kVLoads; ++u)
    {
        const int unit = tid + u * C::kThreads;
        if (unit >= C::kVUnits) break;
        const int quad = unit / C::kRowChunks;
        const int chunk = unit % C::kRowChunks;
        const int pos = vt_pos(quad * 4);  // 4 keys stay contiguous: 8 bytes
        const uint32_t w0[4] = {regs.v[u][0].x, regs.v[u][0].y, regs.v[u][0].z, regs.v[u][0].w};
        const uint32_t w1[4] = {regs.v[u][1].x, regs.v[u][1].y, regs.v[u][1].z, regs.v[u][1].w};
        const uint32_t w2[4] = {regs.v[u][2].x, regs.v[u][2].y, regs.v[u][2].z, regs.v[u][2].w};
        const uint32_t w3[4] = {regs.v[u][3].x, regs.v[u][3].y, regs.v[u][3].z, regs.v[u][3].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
            const int w = e >> 1;
            uint2 out;
            if ((e & 1) == 0)
            {
                out.x = (w0[w] & 0xffffu) | (w1[w] << 16);
                out.y = (w2[w] & 0xffffu) | (w3[w] << 16);
            }
            else
            {
                out.x = (w0[w] >> 16) | (w1[w] & 0xffff0000u);
                out.y = (w2[w] >> 16) | (w3[w] & 0xffff0000u);
            }
            const int dim = chunk * 8 + e;
            *reinterpret_cast<uint2*>(vt_lds + swz<kTileKV>(dim, pos >> 3) + (pos & 7)) = out;
        }
    }
}

// One KV tile for one wave: S^T = K.Q^T, online softmax, O^T += V^T.P^T.
template <int D, bool kCausal, bool kMasked>
__device__ __forceinline__ void tile_step(const uint16_t* k_lds, const uint16_t* vt_lds, const bf16x8 (&qf)[D / 16],
                                          f32x16 (&o)[D / 32], float& m_run, float& l_run, int kv0, int n,
                                          int query, int lane, float c_log2)
{
    const int i = lane & 31;
    const int h = lane >> 5;

    f32x16 s[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
    {
        s[b] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
        {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(k_lds + swz<D>(32 * b + i, 2 * ks + h));
            s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], s[b], 0, 0, 0);
        }
    }

    if (kMasked)
    {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int key = kv0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
                const bool dead = key >= n || (kCausal && key > query);
                if (dead) s[b][r] = -INFINITY;
            }
    }

    float mx = s[0][0];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));

    const float m_new = fmaxf(m_run, mx * c_log2);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;

    float sum = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const float p = __builtin_amdgcn_exp2f(fmaf(s[b][r], c_log2, -m_use));
            s[b][r] = p;
            sum += p;
        }
    l_run = fmaf(l_run, alpha, sum);

#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;

    bf16x8 pf[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[m][e] = static_cast<__bf16>(s[m >> 1][8 * (m & 1) + e]);

#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int m = 0; m < 4; ++m)
        {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(vt_lds + swz<kTileKV>(32 * db + i, 2 * m + h));
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[m], o[db], 0, 0, 0);
        }
}

template <int D, int kWaves, bool kCausal>
__global__ __launch_bounds__(64 * kWaves) void fused_attention_kernel(const uint16_t* __restrict__ q,
                                                                      const uint16_t* __restrict__ k,
                                                                      const uint16_t* __restrict__ v,
                                                                      uint16_t* __restrict__ o, int n,
                                                                      int q_blocks, int total_blocks,
                                                                      float c_log2)
{
    using C = Cfg<D, kWaves>;
    __shared__ __attribute__((aligned(16))) uint16_t lds[C::kLdsElems];
    uint16_t* k_lds = lds;                       // [2][kTileKV][D]
    uint16_t* vt_lds = lds + 2 * C::kKElems;     // [2][D][kTileKV]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int logical = fa::xcd_remap(static_cast<int>(blockIdx.x), total_blocks);
    const int slab = logical / q_blocks;
    const int qb_in = logical % q_blocks;
    const int qb = kCausal ? (q_blocks - 1 - qb_in) : qb_in;  // causal: heaviest first
    const int q0 = qb * C::kRows;
    const int wq0 = q0 + 32 * wave;

    const size_t slab_off = static_cast<size_t>(slab) * n * D;
    const uint16_t* q_slab = q + slab_off;
    const uint16_t* k_slab = k + slab_off;
    const uint16_t* v_slab = v + slab_off;

    const int last_key = kCausal ? min(q0 + C::kRows - 1, n - 1) : n - 1;
    const int n_tiles = last_key / kTileKV + 1;

    // Q rows of this wave as the B operand: lane (j = l%32, h = l/32) holds
    // Q[wq0 + j][16 ks + 8h .. +7] for every K-step ks.
    const int query = wq0 + (lane & 31);
    const int h = lane >> 5;
    bf16x8 qf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
    {
        if (query < n)
            qf[ks] = *reinterpret_cast<const bf16x8*>(q_slab + static_cast<size_t>(query) * D + 16 * ks + 8 * h);
        else
            qf[ks] = bf16x8{};
    }

    f32x16 acc[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) acc[db] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    // Tiles from t_mask on need the per-element mask (sequence tail, or the
    // diagonal for this wave's rows); tiles beyond t_skip lie wholly above
    // this wave's diagonal.
    const int t_tail = (n % kTileKV) ? n / kTileKV : n_tiles;
    const int t_diag = kCausal ? (wq0 + 1) / kTileKV : n_tiles;
    const int t_mask = min(t_tail, t_diag);
    const int t_skip = kCausal ? (wq0 + 31) / kTileKV : n_tiles - 1;  // last tile with work

    TileRegs<D, kWaves> regs;
    load_tile<D, kWaves>(regs, k_slab, v_slab, 0, n, tid);
    store_tile<D, kWaves>(regs, k_lds, vt_lds, tid);
    __syncthreads();

    for (int t = 0; t < n_tiles; ++t)
    {
        const int stage = t & 1;
        const bool has_next = t + 1 < n_tiles;
        if (has_next) load_tile<D, kWaves>(regs, k_slab, v_slab, (t + 1) * kTileKV, n, tid);

        const uint16_t* k_cur = k_lds + stage * C::kKElems;
        const uint16_t* v_cur = vt_lds + stage * C::kVElems;
        if (t <= t_skip)
        {
            if (t < t_mask)
                tile_step<D, kCausal, false>(k_cur, v_cur, qf, acc, m_run, l_run, t * kTileKV, n, query, lane, c_log2);
            else
                tile_step<D, kCausal, true>(k_cur, v_cur, qf, acc, m_run, l_run, t * kTileKV, n, query, lane, c_log2);
        }

        if (has_next)
            store_tile<D, kWaves>(regs, k_lds + (stage ^ 1) * C::kKElems, vt_lds + (stage ^ 1) * C::kVElems, tid);
        __syncthreads();
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
                packed.x = fa::pack_bf16x2(acc[db][4 * g + 0] * inv, acc[db][4 * g + 1] * inv);
                packed.y = fa::pack_bf16x2(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(o_row + 32 * db + 8 * g + 4 * h) = packed;
            }
    }
}

template <int D, int kWaves, bool kCausal>
const void* kernel_ptr()
{
    return reinterpret_cast<const void*>(&fused_attention_kernel<D, kWaves, kCausal>);
}

template <int kWaves>
const void* pick_kernel(int head_dim, bool causal)
{
    if (head_dim == 64) return causal ? kernel_ptr<64, kWaves, true>() : kernel_ptr<64, kWaves, false>();
    if (head_dim == 128) return causal ? kernel_ptr<128, kWaves, true>() : kernel_ptr<128, kWaves, false>();
    return nullptr;
}

template <int D, int kWaves, bool kCausal>
void launch_typed(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int n, int q_blocks,
                  int total, float c_log2, hipStream_t stream)
{
    hipLaunchKernelGGL((fused_attention_kernel<D, kWaves, kCausal>), dim3(static_cast<unsigned>(total)),
                       dim3(Cfg<D, kWaves>::kThreads), 0, stream, q, k, v, o, n, q_blocks, total, c_log2);
}

template <int kWaves>
int launch_fused(const void* q, const void* k, const void* v, void* o, int batch, int heads, int seq_len,
                 int head_dim, int causal, void* stream_ptr)
{
    if (head_dim != 64 && head_dim != 128) return FA_ERROR_UNSUPPORTED;
    if (batch < 0 || heads < 0 || seq_len < 0) return hipErrorInvalidValue;
    const long long bh = static_cast<long long>(batch) * heads;
    if (bh == 0 || seq_len == 0) return hipSuccess;
    if (!q || !k || !v || !o) return hipErrorInvalidValue;
    // 16-byte vector loads and 8-byte stores need aligned bases.
    const uintptr_t mis = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
    if (mis & 15u) return hipErrorInvalidValue;
    constexpr int rows = 32 * kWaves;
    const long long q_blocks = (static_cast<long long>(seq_len) + rows - 1) / rows;
    const long long total = bh * q_blocks;
    if (total > 0x7fffffffLL / (64 * kWaves)) return hipErrorInvalidValue;
    if (bh * seq_len * head_dim > (1LL << 62)) return hipErrorInvalidValue;

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
        if (causal) launch_typed<64, kWaves, true>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
        else launch_typed<64, kWaves, false>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
    }
    else
    {
        if (causal) launch_typed<128, kWaves, true>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
        else launch_typed<128, kWaves, false>(qb, kb, vb, ob, seq_len, qbk, tot, c_log2, stream);
    }
    return static_cast<int>(hipGetLastError());
}

template <int kWaves>
int query_fused(int head_dim, fa_tiling_info* info)
{
    if (!info) return hipErrorInvalidValue;
    *info = fa_tiling_info{};
    if (head_dim != 64 && head_dim != 128) return hipSuccess;  // supported = 0
    info->supported = 1;
    info->block_size = 64 * kWaves;
    info->waves_per_block = kWaves;
    info->tile_kv = kTileKV;
    info->rows_per_block = 32 * kWaves;

    const void* func = pick_kernel<kWaves>(head_dim, false);
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, func);
    if (e != hipSuccess) return e;
    info->shared_bytes_per_block = static_cast<int>(attr.sharedSizeBytes);
    info->registers_per_thread = attr.numRegs;
    info->local_bytes_per_thread = static_cast<int>(attr.localSizeBytes);

    int blocks = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, func, 64 * kWaves, 0);
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
    // hipFuncAttributes has no AGPR field; the kernels keep their MFMA
    // accumulators in ordinary VGPRs (reported above), so this stays 0.
    info->agprs_per_thread = 0;
    return hipSuccess;
}

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
