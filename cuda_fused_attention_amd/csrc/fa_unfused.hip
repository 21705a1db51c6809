// v0: the unfused attention baseline on gfx950 — three kernels with the fp32
// score matrix materialised in HBM, following the reference's algorithm
// (kernels/v0_unfused.cu:19-155): S = scale * Q.K^T in fp32 scalar FMAs
// (masked entries -FLT_MAX), a stable row softmax in place, O = bf16(P.V)
// summed over every key in order.
//
// What is MI355X-specific is the memory access, not the arithmetic:
//   * scores / PV stage 64x32 operand tiles through LDS with 16-byte global
//     loads, so every HBM byte is fetched once per tile and stores are
//     float4 / 8-byte rows (the reference reads K rows per thread, strided);
//   * each thread owns a 4x4 register micro-tile (256 threads -> 64x64 tile);
//   * softmax keeps a whole row in registers (up to 8192 columns), so S is
//     read once and written once — 16 B of HBM traffic per score in total
//     (write S, read S, write P, read P) against the reference's 5 passes.
// Algorithmic bytes per launch: 16*B*H*N^2 + 8*B*H*N*D (HBM roofline).

#include <atomic>
#include <cfloat>
#include <cstdint>

#include "fa_common.hpp"
#include "../../include/fa_mi355x.h"

namespace {

constexpr int kTile = 64;        // outputs per tile edge
constexpr int kChunk = 32;       // reduction chunk staged in LDS
constexpr int kThreads = 256;    // 16 x 16 threads, 4 x 4 outputs each
constexpr int kLdsPitch = kTile + 4;  // floats; 272-byte rows keep float4 alignment

// Load 8 consecutive bf16 (row `row`, columns col..col+7) as floats, zero
// outside [0, rows) x [0, cols). kVec requires cols % 8 == 0 and a 16-byte
// aligned base, so an in-range chunk is one 16-byte load.
template <bool kVec>
__device__ __forceinline__ void load8_bf16(const uint16_t* __restrict__ base, int row, int col, int rows,
                                           int cols, float out[8])
{
    if (kVec)
    {
        if (row < rows && col < cols)
        {
            const uint4 w = *reinterpret_cast<const uint4*>(base + static_cast<size_t>(row) * cols + col);
            out[0] = fa::bf16_lo(w.x); out[1] = fa::bf16_hi(w.x);
            out[2] = fa::bf16_lo(w.y); out[3] = fa::bf16_hi(w.y);
            out[4] = fa::bf16_lo(w.z); out[5] = fa::bf16_hi(w.z);
            out[6] = fa::bf16_lo(w.w); out[7] = fa::bf16_hi(w.w);
        }
        else
        {
#pragma unroll
            for (int e = 0; e < 8; ++e) out[e] = 0.0f;
        }
    }
    else
    {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            out[e] = (row < rows && col + e < cols)
                         ? fa::bf16_bits_to_float(base[static_cast<size_t>(row) * cols + col + e])
                         : 0.0f;
    }
}

// S[bh][q][k] = scale * sum_d Q[q][d] K[k][d]; causal k > q -> -FLT_MAX.
// Grid: (tiles_q * tiles_k, B*H); 256 threads; one 64x64 tile per workgroup.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void v0_scores_kernel(const uint16_t* __restrict__ q,
                                                              const uint16_t* __restrict__ k,
                                                              float* __restrict__ s, int n, int d,
                                                              int tiles_k, float scale, int causal)
{
    __shared__ __attribute__((aligned(16))) float qs[kChunk][kLdsPitch];
    __shared__ __attribute__((aligned(16))) float ks[kChunk][kLdsPitch];

    const int q0 = (blockIdx.x / tiles_k) * kTile;
    const int k0 = (blockIdx.x % tiles_k) * kTile;
    const size_t bh = blockIdx.y;
    const uint16_t* q_slab = q + bh * n * d;
    const uint16_t* k_slab = k + bh * n * d;
    float* s_slab = s + bh * n * n;

    const int tid = threadIdx.x;
    const int tx = tid & 15;   // key micro-column
    const int ty = tid >> 4;   // query micro-row

    if (causal && k0 > q0 + kTile - 1)
    {
        // The whole tile lies above the diagonal: no loads, just the mask.
        for (int i = 0; i < 4; ++i)
        {
            const int query = q0 + ty * 4 + i;
            if (query >= n) break;
            for (int j = 0; j < 4; ++j)
            {
                const int key = k0 + tx * 4 + j;
                if (key < n) s_slab[static_cast<size_t>(query) * n + key] = -FLT_MAX;
            }
        }
        return;
    }

    float acc[4][4] = {};
    const int stage_row = tid >> 2;        // 0..63
    const int stage_col = (tid & 3) * 8;   // 0, 8, 16, 24

    for (int d0 = 0; d0 < d; d0 += kChunk)
    {
        float vals[8];
        load8_bf16<kVec>(q_slab, q0 + stage_row, d0 + stage_col, n, d, vals);
#pragma unroll
        for (int e = 0; e < 8; ++e) qs[stage_col + e][stage_row] = vals[e];
        load8_bf16<kVec>(k_slab, k0 + stage_row, d0 + stage_col, n, d, vals);
#pragma unroll
        for (int e = 0; e < 8; ++e) ks[stage_col + e][stage_row] = vals[e];
        __syncthreads();

#pragma unroll 8
        for (int dd = 0; dd < kChunk; ++dd)
        {
            const float4 a = *reinterpret_cast<const float4*>(&qs[dd][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&ks[dd][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w};
            const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }

    const bool full_cols = (k0 + tx * 4 + 3 < n) && ((n & 3) == 0);
    for (int i = 0; i < 4; ++i)
    {
        const int query = q0 + ty * 4 + i;
        if (query >= n) break;
        float out[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int key = k0 + tx * 4 + j;
            out[j] = (causal && key > query) ? -FLT_MAX : acc[i][j] * scale;
        }
        float* dst = s_slab + static_cast<size_t>(query) * n + k0 + tx * 4;
        if (full_cols)
            *reinterpret_cast<float4*>(dst) = make_float4(out[0], out[1], out[2], out[3]);
        else
            for (int j = 0; j < 4; ++j)
                if (k0 + tx * 4 + j < n) dst[j] = out[j];
    }
}

__device__ __forceinline__ float block_reduce_max(float x, float* scratch)
{
    x = fa::wave_max(x);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = x;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, scratch[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_reduce_sum(float x, float* scratch)
{
    x = fa::wave_sum(x);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = x;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < kThreads / 64; ++w) r += scratch[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float softmax_exp(float x, float row_max)
{
    return __builtin_amdgcn_exp2f((x - row_max) * fa::kLog2e);
}

// One workgroup per row; the row lives in registers (kVecs float4 per
// thread, cols <= 1024 * kVecs, cols % 4 == 0, 16-byte aligned base):
// read once, write once. Same stages as kernels/v0_unfused.cu:51-94: max,
// exp(x - max) and sum, multiply by 1/sum (sum <= 0 -> 1).
template <int kVecs>
__global__ __launch_bounds__(kThreads) void v0_softmax_rows_reg_kernel(float* __restrict__ s, int cols)
{
    __shared__ float scratch[kThreads / 64];
    float4* row = reinterpret_cast<float4*>(s + static_cast<size_t>(blockIdx.x) * cols);
    const int nvec = cols >> 2;

    float4 v[kVecs];
    float local_max = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < kVecs; ++i)
    {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nvec)
        {
            v[i] = row[idx];
            local_max = fmaxf(local_max, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
        }
    }
    const float row_max = block_reduce_max(local_max, scratch);

    float local_sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kVecs; ++i)
    {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nvec)
        {
            v[i].x = softmax_exp(v[i].x, row_max);
            v[i].y = softmax_exp(v[i].y, row_max);
            v[i].z = softmax_exp(v[i].z, row_max);
            v[i].w = softmax_exp(v[i].w, row_max);
            local_sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        }
    }
    const float total = block_reduce_sum(local_sum, scratch);
    const float inverse = 1.0f / (total > 0.0f ? total : 1.0f);

#pragma unroll
    for (int i = 0; i < kVecs; ++i)
    {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nvec)
            row[idx] = make_float4(v[i].x * inverse, v[i].y * inverse, v[i].z * inverse, v[i].w * inverse);
    }
}

// Any cols and alignment: the reference's three passes over the row in HBM.
__global__ __launch_bounds__(kThreads) void v0_softmax_rows_loop_kernel(float* __restrict__ s, int cols)
{
    __shared__ float scratch[kThreads / 64];
    float* row = s + static_cast<size_t>(blockIdx.x) * cols;
    float local_max = -FLT_MAX;
    for (int c = threadIdx.x; c < cols; c += kThreads) local_max = fmaxf(local_max, row[c]);
    const float row_max = block_reduce_max(local_max, scratch);
    float local_sum = 0.0f;
    for (int c = threadIdx.x; c < cols; c += kThreads)
    {
        const float e = softmax_exp(row[c], row_max);
        row[c] = e;
        local_sum += e;
    }
    const float total = block_reduce_sum(local_sum, scratch);
    const float inverse = 1.0f / (total > 0.0f ? total : 1.0f);
    for (int c = threadIdx.x; c < cols; c += kThreads) row[c] *= inverse;
}

// O[bh][q][d] = bf16_rne(sum_k P[q][k] V[k][d]), keys in order 0..n-1.
// Grid: (tiles_q * tiles_d, B*H); 256 threads; one 64 x 64 output tile.
// kVec requires n % 8 == 0, d % 8 == 0 and 16-byte aligned bases.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void v0_pv_kernel(const float* __restrict__ p,
                                                          const uint16_t* __restrict__ v,
                                                          uint16_t* __restrict__ o, int n, int d,
                                                          int tiles_d)
{
    __shared__ __attribute__((aligned(16))) float ps[kChunk][kLdsPitch];  // [key][query]
    __shared__ __attribute__((aligned(16))) float vs[kChunk][kLdsPitch];  // [key][dim]

    const int q0 = (blockIdx.x / tiles_d) * kTile;
    const int c0 = (blockIdx.x % tiles_d) * kTile;
    const size_t bh = blockIdx.y;
    const float* p_slab = p + bh * n * n;
    const uint16_t* v_slab = v + bh * n * d;
    uint16_t* o_slab = o + bh * n * d;

    const int tid = threadIdx.x;
    const int tx = tid & 15;
    const int ty = tid >> 4;
    const int p_row = tid >> 2;         // query within tile
    const int p_col = (tid & 3) * 8;    // key within chunk
    const int v_row = tid >> 3;         // key within chunk
    const int v_col = (tid & 7) * 8;    // dim within tile

    float acc[4][4] = {};
    for (int k0 = 0; k0 < n; k0 += kChunk)
    {
        const int query = q0 + p_row;
        float pv[8];
        if (kVec)
        {
            if (query < n && k0 + p_col < n)
            {
                const float4* src = reinterpret_cast<const float4*>(p_slab + static_cast<size_t>(query) * n + k0 + p_col);
                const float4 a = src[0];
                const float4 b = src[1];
                pv[0] = a.x; pv[1] = a.y; pv[2] = a.z; pv[3] = a.w;
                pv[4] = b.x; pv[5] = b.y; pv[6] = b.z; pv[7] = b.w;
            }
            else
            {
#pragma unroll
                for (int e = 0; e < 8; ++e) pv[e] = 0.0f;
            }
        }
        else
        {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                pv[e] = (query < n && k0 + p_col + e < n) ? p_slab[static_cast<size_t>(query) * n + k0 + p_col + e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ps[p_col + e][p_row] = pv[e];

        float vv[8];
        load8_bf16<kVec>(v_slab, k0 + v_row, c0 + v_col, n, d, vv);
        *reinterpret_cast<float4*>(&vs[v_row][v_col]) = make_float4(vv[0], vv[1], vv[2], vv[3]);
        *reinterpret_cast<float4*>(&vs[v_row][v_col + 4]) = make_float4(vv[4], vv[5], vv[6], vv[7]);
        __syncthreads();

#pragma unroll 8
        for (int kk = 0; kk < kChunk; ++kk)
        {
            const float4 a = *reinterpret_cast<const float4*>(&ps[kk][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&vs[kk][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w};
            const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }

    const int col = c0 + tx * 4;
    for (int i = 0; i < 4; ++i)
    {
        const int query = q0 + ty * 4 + i;
        if (query >= n) break;
        uint16_t* dst = o_slab + static_cast<size_t>(query) * d + col;
        if (kVec && col + 3 < d)
        {
            uint2 packed;
            packed.x = fa::pack_bf16x2(acc[i][0], acc[i][1]);
            packed.y = fa::pack_bf16x2(acc[i][2], acc[i][3]);
            *reinterpret_cast<uint2*>(dst) = packed;
        }
        else
        {
            for (int j = 0; j < 4; ++j)
                if (col + j < d) dst[j] = fa::float_to_bf16_bits(acc[i][j]);
        }
    }
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

constexpr int kMaxGridY = 65535;

int launch_softmax(float* s, int rows, int cols, hipStream_t stream)
{
    const dim3 grid(static_cast<unsigned>(rows));
    const dim3 block(kThreads);
    const bool vec = (cols % 4 == 0) && aligned16(s);
    if (vec && cols <= 1024 * 1) return fa::launch_kernel(v0_softmax_rows_reg_kernel<1>, grid, block, stream, s, cols);
    if (vec && cols <= 1024 * 2) return fa::launch_kernel(v0_softmax_rows_reg_kernel<2>, grid, block, stream, s, cols);
    if (vec && cols <= 1024 * 4) return fa::launch_kernel(v0_softmax_rows_reg_kernel<4>, grid, block, stream, s, cols);
    if (vec && cols <= 1024 * 8) return fa::launch_kernel(v0_softmax_rows_reg_kernel<8>, grid, block, stream, s, cols);
    return fa::launch_kernel(v0_softmax_rows_loop_kernel, grid, block, stream, s, cols);
}

// Shape and pointer checks shared by the v0 entry points (the workspace is
// checked by the caller): hipSuccess, -1 for an empty shape (nothing to
// launch) or hipErrorInvalidValue.
int validate_unfused(const void* q, const void* k, const void* v, void* o, int batch, int heads, int seq_len,
                     int head_dim)
{
    if (batch < 0 || heads < 0 || seq_len < 0 || head_dim <= 0) return hipErrorInvalidValue;
    const long long bh = static_cast<long long>(batch) * heads;
    if (bh == 0 || seq_len == 0) return -1;  // empty: nothing to launch
    if (!q || !k || !v || !o) return hipErrorInvalidValue;
    if (bh > kMaxGridY) return hipErrorInvalidValue;
    const long long tiles = (static_cast<long long>(seq_len) + kTile - 1) / kTile;
    if (tiles * tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    if (bh * seq_len > 0x7fffffffLL) return hipErrorInvalidValue;  // softmax grid
    return hipSuccess;
}

int launch_unfused_impl(const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
                        int heads, int seq_len, int head_dim, int causal, hipEvent_t const* events,
                        hipStream_t stream)
{
    const int status = validate_unfused(q, k, v, o, batch, heads, seq_len, head_dim);
    if (status == -1) return hipSuccess;
    if (status != hipSuccess) return status;
    if (!workspace) return hipErrorInvalidValue;

    const int bh = batch * heads;
    const int n = seq_len;
    const int d = head_dim;
    const float scale = fa_default_scale(d);
    const uint16_t* qb = static_cast<const uint16_t*>(q);
    const uint16_t* kb = static_cast<const uint16_t*>(k);
    const uint16_t* vb = static_cast<const uint16_t*>(v);
    uint16_t* ob = static_cast<uint16_t*>(o);
    const int tiles_n = (n + kTile - 1) / kTile;
    const int tiles_d = (d + kTile - 1) / kTile;

    if (events)
    {
        const hipError_t e = hipEventRecord(events[0], stream);
        if (e != hipSuccess) return e;
    }
    const bool vec_qk = (d % 8 == 0) && aligned16(q) && aligned16(k);
    const dim3 grid_s(static_cast<unsigned>(tiles_n * tiles_n), static_cast<unsigned>(bh));
    hipError_t e = fa::launch_kernel(vec_qk ? v0_scores_kernel<true> : v0_scores_kernel<false>, grid_s,
                                     dim3(kThreads), stream, qb, kb, workspace, n, d, tiles_n, scale, causal);
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[1], stream)) != hipSuccess) return e;

    // The softmax sees the workspace as one [B*H*N, N] matrix.
    e = static_cast<hipError_t>(launch_softmax(workspace, bh * n, n, stream));
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[2], stream)) != hipSuccess) return e;

    const bool vec_pv = (n % 8 == 0) && (d % 8 == 0) && aligned16(workspace) && aligned16(v) && aligned16(o);
    const dim3 grid_o(static_cast<unsigned>(tiles_n * tiles_d), static_cast<unsigned>(bh));
    e = fa::launch_kernel(vec_pv ? v0_pv_kernel<true> : v0_pv_kernel<false>, grid_o, dim3(kThreads), stream,
                          workspace, vb, ob, n, d, tiles_d);
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[3], stream)) != hipSuccess) return e;
    return hipSuccess;
}

// The allocation-free v0 entry point's score workspace: a file-scope device
// array, one copy per GPU, held for the life of the process. In host code
// its name is only a stand-in for the symbol; the device address is looked
// up once per device (noalloc_scratch) and only that address is used.
constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;
__device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device (hipGetSymbolAddress,
// once per device, cached), or null with the HIP status in *status.
float* noalloc_scratch(int* status)
{
    static std::atomic<uintptr_t> cache[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    {
        *status = e != hipSuccess ? e : hipErrorInvalidDevice;
        return nullptr;
    }
    uintptr_t addr = cache[dev].load(std::memory_order_acquire);
    if (addr == 0)
    {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
        {
            *status = e != hipSuccess ? e : hipErrorInvalidSymbol;
            return nullptr;
        }
        addr = reinterpret_cast<uintptr_t>(ptr);
        cache[dev].store(addr, std::memory_order_release);
    }
    *status = hipSuccess;
    return reinterpret_cast<float*>(addr);
}

int launch_unfused_noalloc(const void* q, const void* k, const void* v, void* o, int batch, int heads, int seq_len,
                           int head_dim, int causal, hipStream_t stream)
{
    // The same checks as the workspace entry, minus the workspace pointer.
    int status = validate_unfused(q, k, v, o, batch, heads, seq_len, head_dim);
    if (status == -1) return hipSuccess;
    if (status != hipSuccess) return status;
    const size_t need = fa_unfused_workspace_bytes(batch, heads, seq_len, head_dim);
    if (need > kNoAllocScratchBytes) return hipErrorInvalidValue;
    float* ws = noalloc_scratch(&status);
    if (!ws) return status;
    // The scores kernel writes every element of S the softmax and PV kernels
    // read (masked ones as -FLT_MAX), so the array needs no clearing between
    // calls.
    return launch_unfused_impl(q, k, v, o, ws, batch, heads, seq_len, head_dim, causal, nullptr, stream);
}

}  // namespace

extern "C" {

size_t fa_unfused_noalloc_max_workspace_bytes(void) { return kNoAllocScratchBytes; }

int fa_launch_attention_unfused_noalloc(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                                        int seq_len, int head_dim, int causal, void* stream)
{
    return fa::record_status(launch_unfused_noalloc(q, k, v, o, batch, heads, seq_len, head_dim, causal,
                                                    static_cast<hipStream_t>(stream)));
}

float fa_default_scale(int head_dim) { return 1.0f / sqrtf(static_cast<float>(head_dim)); }

double fa_attention_flops(int batch, int heads, int seq_len, int head_dim, int causal)
{
    const double n = static_cast<double>(seq_len);
    const double pairs = causal ? n * (n + 1.0) / 2.0 : n * n;
    return 4.0 * pairs * static_cast<double>(head_dim) * static_cast<double>(batch) * static_cast<double>(heads);
}

size_t fa_unfused_workspace_bytes(int batch, int heads, int seq_len, int /*head_dim*/)
{
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;
    return static_cast<size_t>(batch) * heads * seq_len * static_cast<size_t>(seq_len) * sizeof(float);
}

int fa_launch_softmax_rows_inplace(float* s, int rows, int cols, void* stream)
{
    if (rows < 0 || cols < 0) return fa::record_status(hipErrorInvalidValue);
    if (rows == 0 || cols == 0) return hipSuccess;
    if (!s) return fa::record_status(hipErrorInvalidValue);
    return fa::record_status(launch_softmax(s, rows, cols, static_cast<hipStream_t>(stream)));
}

int fa_launch_attention_unfused(const void* q, const void* k, const void* v, void* o, float* workspace,
                                int batch, int heads, int seq_len, int head_dim, int causal, void* stream)
{
    return fa::record_status(launch_unfused_impl(q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal,
                                                 nullptr, static_cast<hipStream_t>(stream)));
}

int fa_launch_attention_unfused_profile(const void* q, const void* k, const void* v, void* o, float* workspace,
                                        int batch, int heads, int seq_len, int head_dim, int causal,
                                        void* const* events, void* stream)
{
    return fa::record_status(launch_unfused_impl(q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal,
                                                 reinterpret_cast<hipEvent_t const*>(events),
                                                 static_cast<hipStream_t>(stream)));
}

}  // extern "C"
