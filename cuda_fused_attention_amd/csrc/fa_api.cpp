// C++ launch interface of include/flash_attention.h (the reference's
// namespace cuda_op_lab::flash_attention, include/flash_attention.h:9-109)
// implemented over the C ABI of include/fa_mi355x.h, plus the hipEvent timing
// entry points (benchmarks/bench_flash_attention.cu:265-299 semantics).

#include <hip/hip_runtime.h>

#include <cmath>

#include "../../include/fa_mi355x.h"
#include "../../include/flash_attention.h"
#include "../../include/flash_attention_v0_profile.h"
#include "fa_common.hpp"

namespace {

// The calling thread's last non-success status of a C-ABI call
// (fa_get_last_error / fa_peek_at_last_error; hipGetLastError semantics).
thread_local int t_last_status = 0;

}  // namespace

namespace fa {

int record_status(int status)
{
    if (status != 0 && status != FA_ERROR_UNSUPPORTED) t_last_status = status;
    return status;
}

}  // namespace fa

namespace cuda_op_lab::flash_attention {

hipError_t get_last_error() { return static_cast<hipError_t>(fa_get_last_error()); }

hipError_t peek_at_last_error() { return static_cast<hipError_t>(fa_peek_at_last_error()); }

namespace {

FusedTilingInfo to_cpp(const fa_tiling_info& c)
{
    FusedTilingInfo info{};
    info.supported = c.supported != 0;
    info.block_size = c.block_size;
    info.tile_kv = c.tile_kv;
    info.rows_per_block = c.rows_per_block;
    info.shared_bytes_per_block = c.shared_bytes_per_block;
    info.registers_per_thread = c.registers_per_thread;
    info.local_bytes_per_thread = c.local_bytes_per_thread;
    info.max_blocks_per_sm = c.max_blocks_per_sm;
    info.device_shared_bytes_per_sm = c.device_shared_bytes_per_sm;
    info.shared_limited_blocks_per_sm = c.shared_limited_blocks_per_sm;
    return info;
}

}  // namespace

// The launchers return void, as the reference's do; a non-zero status of
// the C-ABI call under them is kept per thread for get_last_error().

double attention_flops(const AttentionShape& s, bool causal)
{
    return fa_attention_flops(s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0);
}

size_t unfused_workspace_bytes(const AttentionShape& s)
{
    return fa_unfused_workspace_bytes(s.batch, s.heads, s.seq_len, s.head_dim);
}

void launch_attention_unfused(const __hip_bfloat16* q, const __hip_bfloat16* k, const __hip_bfloat16* v,
                              __hip_bfloat16* o, float* workspace, const AttentionShape& s, bool causal,
                              hipStream_t stream)
{
    (void)fa_launch_attention_unfused(q, k, v, o, workspace, s.batch, s.heads, s.seq_len, s.head_dim,
                                      causal ? 1 : 0, stream);
}

void launch_softmax_rows_inplace(float* s, int rows, int cols, hipStream_t stream)
{
    (void)fa_launch_softmax_rows_inplace(s, rows, cols, stream);
}

hipError_t launch_attention_unfused_profile(const __hip_bfloat16* q, const __hip_bfloat16* k,
                                            const __hip_bfloat16* v, __hip_bfloat16* o, float* workspace,
                                            const AttentionShape& s, bool causal, const V0ProfileEvents* events,
                                            hipStream_t stream)
{
    void* handles[4];
    void* const* ev = nullptr;
    if (events)
    {
        handles[0] = events->qk_start;
        handles[1] = events->qk_end;
        handles[2] = events->softmax_end;
        handles[3] = events->pv_end;
        ev = handles;
    }
    return static_cast<hipError_t>(fa_launch_attention_unfused_profile(
        q, k, v, o, workspace, s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0, ev, stream));
}

// v1 / v2 / v2b study kernels are not rebuilt for gfx950 (see header).
bool fused_row_supported(int) { return false; }

void launch_attention_fused_row(const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*,
                                __hip_bfloat16*, const AttentionShape&, bool, hipStream_t)
{
}

FusedRowInfo query_fused_row(int) { return FusedRowInfo{}; }

void launch_attention_fusedtiling(const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*,
                                  __hip_bfloat16*, const AttentionShape&, bool, hipStream_t)
{
}

FusedTilingInfo query_fused_tiling(int) { return FusedTilingInfo{}; }

double fused_tiling_hbm_bytes(const AttentionShape&, bool) { return 0.0; }

void launch_attention_fusedtiling_v2b(const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*,
                                      __hip_bfloat16*, const AttentionShape&, bool, hipStream_t)
{
}

FusedTilingInfo query_fused_tiling_v2b(int) { return FusedTilingInfo{}; }

double fused_tiling_v2b_hbm_bytes(const AttentionShape&, bool) { return 0.0; }

bool tensorcore_v3_supported(int head_dim) { return fa_tensorcore_v3_supported(head_dim) != 0; }

void launch_attention_tensorcore_v3(const __hip_bfloat16* q, const __hip_bfloat16* k, const __hip_bfloat16* v,
                                    __hip_bfloat16* o, const AttentionShape& s, bool causal, hipStream_t stream)
{
    (void)fa_launch_attention_tensorcore_v3(q, k, v, o, s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0,
                                            stream);
}

FusedTilingInfo query_tensorcore_v3(int head_dim)
{
    fa_tiling_info c{};
    if (fa_query_tensorcore_v3(head_dim, &c) != 0) return FusedTilingInfo{};
    return to_cpp(c);
}

FusedTilingInfo query_tensorcore_v3(const AttentionShape& s, bool causal)
{
    fa_tiling_info c{};
    if (fa_query_tensorcore_v3_shape(s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0, &c) != 0)
        return FusedTilingInfo{};
    return to_cpp(c);
}

double tensorcore_v3_hbm_bytes(const AttentionShape& s, bool causal)
{
    return fa_tensorcore_v3_hbm_bytes(s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0);
}

bool tensorcore_v3b_supported(int head_dim) { return fa_tensorcore_v3b_supported(head_dim) != 0; }

void launch_attention_tensorcore_v3b(const __hip_bfloat16* q, const __hip_bfloat16* k, const __hip_bfloat16* v,
                                     __hip_bfloat16* o, const AttentionShape& s, bool causal, hipStream_t stream)
{
    (void)fa_launch_attention_tensorcore_v3b(q, k, v, o, s.batch, s.heads, s.seq_len, s.head_dim,
                                             causal ? 1 : 0, stream);
}

FusedTilingInfo query_tensorcore_v3b(int head_dim)
{
    fa_tiling_info c{};
    if (fa_query_tensorcore_v3b(head_dim, &c) != 0) return FusedTilingInfo{};
    return to_cpp(c);
}

double tensorcore_v3b_hbm_bytes(const AttentionShape& s, bool causal)
{
    return fa_tensorcore_v3b_hbm_bytes(s.batch, s.heads, s.seq_len, s.head_dim, causal ? 1 : 0);
}

}  // namespace cuda_op_lab::flash_attention

namespace {

int launch_which(int which, const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
                 int heads, int seq_len, int head_dim, int causal, void* stream)
{
    switch (which)
    {
        case 0: return fa_launch_attention_unfused(q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal, stream);
        case 1: return fa_launch_attention_tensorcore_v3(q, k, v, o, batch, heads, seq_len, head_dim, causal, stream);
        case 2: return fa_launch_attention_tensorcore_v3b(q, k, v, o, batch, heads, seq_len, head_dim, causal, stream);
        case 3: return fa_launch_attention_fused(q, k, v, o, batch, heads, seq_len, head_dim, causal, 128, stream);
        case 4: return fa_launch_attention_fused(q, k, v, o, batch, heads, seq_len, head_dim, causal, 256, stream);
        case 5:
            return fa_launch_attention_fused_groups(q, k, v, o, batch, heads, seq_len, head_dim, causal, 64, 4, stream);
        case 6:
            return fa_launch_attention_fused_groups(q, k, v, o, batch, heads, seq_len, head_dim, causal, 128, 4, stream);
        default: return hipErrorInvalidValue;
    }
}

struct EventPair
{
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    ~EventPair()
    {
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
    }
};

}  // namespace

extern "C" {

int fa_get_last_error(void)
{
    const int status = t_last_status;
    t_last_status = 0;
    return status;
}

int fa_peek_at_last_error(void) { return t_last_status; }

namespace {

int time_launches(int which, const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
                  int heads, int seq_len, int head_dim, int causal, int warmup, int iters, float* samples_ms,
                  void* stream)
{
    if (warmup < 0 || iters <= 0 || !samples_ms) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < warmup; ++i)
    {
        const int e = launch_which(which, q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal, stream);
        if (e != 0) return e;
    }
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;

    EventPair ev;
    if ((e = hipEventCreate(&ev.start)) != hipSuccess) return e;
    if ((e = hipEventCreate(&ev.stop)) != hipSuccess) return e;
    for (int i = 0; i < iters; ++i)
    {
        if ((e = hipEventRecord(ev.start, s)) != hipSuccess) return e;
        const int le = launch_which(which, q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal, stream);
        if (le != 0) return le;
        if ((e = hipEventRecord(ev.stop, s)) != hipSuccess) return e;
        if ((e = hipEventSynchronize(ev.stop)) != hipSuccess) return e;
        float ms = 0.0f;
        if ((e = hipEventElapsedTime(&ms, ev.start, ev.stop)) != hipSuccess) return e;
        if (!std::isfinite(ms) || ms <= 0.0f) return hipErrorInvalidValue;
        samples_ms[i] = ms;
    }
    return hipSuccess;
}

int time_batch(int which, const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
               int heads, int seq_len, int head_dim, int causal, int iters, float* total_ms, void* stream)
{
    if (iters <= 0 || !total_ms) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    EventPair ev;
    hipError_t e;
    if ((e = hipEventCreate(&ev.start)) != hipSuccess) return e;
    if ((e = hipEventCreate(&ev.stop)) != hipSuccess) return e;
    if ((e = hipEventRecord(ev.start, s)) != hipSuccess) return e;
    for (int i = 0; i < iters; ++i)
    {
        const int le = launch_which(which, q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal, stream);
        if (le != 0) return le;
    }
    if ((e = hipEventRecord(ev.stop, s)) != hipSuccess) return e;
    if ((e = hipEventSynchronize(ev.stop)) != hipSuccess) return e;
    float ms = 0.0f;
    if ((e = hipEventElapsedTime(&ms, ev.start, ev.stop)) != hipSuccess) return e;
    if (!std::isfinite(ms) || ms <= 0.0f) return hipErrorInvalidValue;
    *total_ms = ms;
    return hipSuccess;
}

}  // namespace

int fa_time_launches(int which, const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
                     int heads, int seq_len, int head_dim, int causal, int warmup, int iters, float* samples_ms,
                     void* stream)
{
    return fa::record_status(time_launches(which, q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal,
                                           warmup, iters, samples_ms, stream));
}

int fa_time_batch(int which, const void* q, const void* k, const void* v, void* o, float* workspace, int batch,
                  int heads, int seq_len, int head_dim, int causal, int iters, float* total_ms, void* stream)
{
    return fa::record_status(time_batch(which, q, k, v, o, workspace, batch, heads, seq_len, head_dim, causal, iters,
                                        total_ms, stream));
}

const char* fa_build_info(void)
{
    return "libfa_mi355x gfx950: v0 unfused (fp32 SIMT, LDS-tiled) + fused v_mfma_f32_32x32x16_bf16 "
           "(32 query rows/wave, 32-key K/V tiles by buffer-load LDS DMA, 3 stages per tensor, MFMA/VALU interleaved per wave; "
           "workgroups of 128 rows (2 split-KV groups x 4 waves), 64 rows (2 x 2, or 4 x 2 at head_dim 64) or "
           "256 rows (1 group x 8 waves), v3 picks by shape)";
}

}  // extern "C"
