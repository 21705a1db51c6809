/*
 * fa_mi355x.h — C ABI of the MI355X (gfx950) BF16 attention forward library
 * (libfa_mi355x.so). Plain pointers and ints only, so ctypes, cgo, JNI or a
 * C harness can bind it without C++ or torch types.
 *
 * Every entry point returns an int status: 0 (hipSuccess) or a hipError_t
 * value. Launchers are asynchronous and stream-ordered on `stream` (a
 * hipStream_t; NULL = the null stream); device-side failures surface on the
 * next synchronisation, as with the reference's launchers. Launchers allocate
 * nothing and keep no state; the caller owns q, k, v, o and the workspace.
 *
 * Tensors are contiguous [batch, heads, seq_len, head_dim] bf16 (IEEE
 * binary16-brain bit patterns, 2 bytes each); accumulation is fp32; the
 * softmax scale is 1/sqrt(head_dim) computed in float
 * (include/flash_attention.h:21-24 of the reference).
 *
 * Error contract (the reference returns void and reports through
 * cudaGetLastError; this layer returns the code directly):
 *   FA_ERROR_UNSUPPORTED   head_dim not handled by that kernel — nothing is
 *                          launched (the reference's launchers return silently
 *                          here, kernels/v3/v3_tensorcore.cu:743-744);
 *   hipErrorInvalidValue   null pointer with a non-empty shape, negative
 *                          dimension, misaligned fused-kernel base, a slab
 *                          past 2^31 bytes, or a shape beyond the grid limits
 *                          (host-side rejections: nothing is launched);
 *   a hipError_t           the runtime refused a kernel launch (the status of
 *                          that launch alone; it also stays in HIP's own
 *                          last-error state, so hipGetLastError sees it);
 *   0 with no launch       any of batch, heads, seq_len equal to 0.
 * Every non-zero status except FA_ERROR_UNSUPPORTED is also kept per thread
 * for fa_get_last_error / fa_peek_at_last_error, which is how a caller of the
 * void C++ launchers of flash_attention.h sees host-side rejections.
 *
 * Reference interface each symbol replaces is cited per declaration
 * (paths relative to the RichterWang/cuda_fused_attention tree).
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ERROR_UNSUPPORTED 801 /* == hipErrorNotSupported */

/* Kernel resource report. Field meaning follows the reference's
 * FusedTilingInfo (include/flash_attention.h:60-72); the last three fields are
 * MI355X additions (AGPRs and the LDS/wave budgets of a gfx950 CU). */
typedef struct fa_tiling_info {
    int supported;
    int block_size;                  /* threads per workgroup */
    int tile_kv;                     /* key/value rows staged in LDS per step */
    int rows_per_block;              /* query rows per workgroup */
    int shared_bytes_per_block;      /* LDS bytes per workgroup */
    int registers_per_thread;        /* VGPRs */
    int local_bytes_per_thread;      /* scratch (spill) bytes, must be 0 */
    int max_blocks_per_sm;           /* workgroups resident per CU */
    int device_shared_bytes_per_sm;  /* LDS per CU */
    int shared_limited_blocks_per_sm;
    int agprs_per_thread;            /* accumulation VGPRs (MI355X), from the
                                        compiler's report; -1 if unknown */
    int waves_per_block;             /* wave64 count per workgroup (MI355X) */
    int compute_units;               /* CUs on the current device (MI355X) */
    int kv_groups;                   /* wave groups splitting the KV range (MI355X) */
} fa_tiling_info;

/* No counterpart in the reference (its launchers return void and leave
 * errors to cudaGetLastError): the calling thread's last non-zero status of
 * an fa_* launcher, query or timing call, FA_ERROR_UNSUPPORTED excepted.
 * fa_get_last_error returns it and resets it to 0 (hipGetLastError
 * semantics); fa_peek_at_last_error leaves it. For callers of the void C++
 * launchers, whose host-side rejections never reach HIP's error state. */
int fa_get_last_error(void);
int fa_peek_at_last_error(void);

/* include/flash_attention.h:21-24 — 1.0f / sqrtf(head_dim). */
float fa_default_scale(int head_dim);

/* include/flash_attention.h:27, kernels/v0_unfused.cu:118-126 — 4*pairs*D*B*H,
 * pairs = N^2 dense, N(N+1)/2 causal (the reference's convention). */
double fa_attention_flops(int batch, int heads, int seq_len, int head_dim, int causal);

/* include/flash_attention.h:30, kernels/v0_unfused.cu:128-131 — B*H*N*N*4. */
size_t fa_unfused_workspace_bytes(int batch, int heads, int seq_len, int head_dim);

/* include/flash_attention.h:33, kernels/v0_unfused.cu:140-155 — the unfused
 * baseline: S = scale*Q.K^T (fp32, masked to -FLT_MAX) into `workspace`
 * (>= fa_unfused_workspace_bytes), row softmax in place, O = bf16(P.V).
 * Three kernels, one stream, no host sync. Any head_dim >= 1. */
int fa_launch_attention_unfused(const void* q, const void* k, const void* v, void* o,
                                float* workspace, int batch, int heads, int seq_len,
                                int head_dim, int causal, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): fa_launch_attention_unfused without the workspace
 * argument. The score workspace is a 64 MiB array inside the library, one
 * per GPU, held until the process ends; shapes needing more
 * (fa_unfused_workspace_bytes > fa_unfused_noalloc_max_workspace_bytes(),
 * e.g. B*H*N*N > 16M) return hipErrorInvalidValue and launch nothing. It
 * calls no allocator. Every call on one GPU uses that GPU's one array:
 * calls that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller. Same kernels, so the same output bits as the
 * workspace entry. */
int fa_launch_attention_unfused_noalloc(const void* q, const void* k, const void* v, void* o,
                                        int batch, int heads, int seq_len, int head_dim,
                                        int causal, void* stream);
size_t fa_unfused_noalloc_max_workspace_bytes(void);

/* include/flash_attention.h:36, kernels/v0_unfused.cu:133-138 — stable row
 * softmax in place over a [rows, cols] fp32 matrix. */
int fa_launch_softmax_rows_inplace(float* s, int rows, int cols, void* stream);

/* include/flash_attention_v0_profile.h:9-23, kernels/v0_unfused_profile.cu:121-148
 * — the same three kernels with four hipEvent_t markers recorded on `stream`
 * (qk_start, qk_end, softmax_end, pv_end). `events` may be NULL (no markers);
 * otherwise it points at four hipEvent_t handles in that order. */
int fa_launch_attention_unfused_profile(const void* q, const void* k, const void* v, void* o,
                                        float* workspace, int batch, int heads, int seq_len,
                                        int head_dim, int causal, void* const* events,
                                        void* stream);

/* include/flash_attention.h:90 — head_dim in {64, 128}. */
int fa_tensorcore_v3_supported(int head_dim);

/* include/flash_attention.h:92, kernels/v3/v3_tensorcore.cu:722-750 — the
 * fused forward: QK^T and PV on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16),
 * K and V^T staged in LDS, online softmax in fp32 registers, whole KV tiles
 * above the causal diagonal skipped. 128 query rows per workgroup; a shape
 * whose 128-row grid has fewer workgroups than the device has CUs runs the
 * 64-row configuration instead (fa_launch_attention_fused, rows 0). */
int fa_launch_attention_tensorcore_v3(const void* q, const void* k, const void* v, void* o,
                                      int batch, int heads, int seq_len, int head_dim,
                                      int causal, void* stream);

/* No counterpart in the reference (whose v3 has one tile configuration): the
 * fused forward with an explicit workgroup configuration. rows_per_block is
 * 128 (the v3 configuration: two wave groups split the KV range), 64 (the
 * v3b configuration), 256 (one group of 8 waves walks the whole KV range:
 * half the L2->LDS copies per score, for grids with many workgroups per CU)
 * or 0 (the choice fa_launch_attention_tensorcore_v3 makes); anything else
 * returns hipErrorInvalidValue. For callers and tests that pin the
 * configuration. */
int fa_launch_attention_fused(const void* q, const void* k, const void* v, void* o,
                              int batch, int heads, int seq_len, int head_dim,
                              int causal, int rows_per_block, void* stream);

/* No counterpart in the reference: the fused forward in any of its workgroup
 * configurations, named by query rows per workgroup and the number of wave
 * groups that split the KV range: (128, 2) is v3's default, (64, 2) v3b,
 * (256, 1) one group of 8 waves, (64, 4) four groups of 2 waves, and
 * (128, 4): two 64-row half blocks whose K/V tiles form one list (the first
 * half block's tiles, then the second's), walked in four quarters by four
 * groups of 2 waves that move to the second half block's rows where their
 * quarter crosses into it; every group works on every step however unequal
 * the half blocks' causal tile counts. The last two exist at head_dim 64
 * only: FA_ERROR_UNSUPPORTED at 128, whose four stage sets would not fit
 * LDS. Other pairs return hipErrorInvalidValue. */
int fa_launch_attention_fused_groups(const void* q, const void* k, const void* v, void* o,
                                     int batch, int heads, int seq_len, int head_dim,
                                     int causal, int rows_per_block, int kv_groups, void* stream);

/* No counterpart in the reference: fa_query_tensorcore_v3 for the
 * configuration fa_launch_attention_fused runs with rows_per_block (64, 128
 * or 256; two groups below 256 rows), or fa_launch_attention_fused_groups
 * with (rows_per_block, kv_groups). agprs_per_thread comes from the compiler's resource report of
 * the kernel, recorded when the library was built. */
int fa_query_fused(int head_dim, int rows_per_block, fa_tiling_info* info);
int fa_query_fused_groups(int head_dim, int rows_per_block, int kv_groups, fa_tiling_info* info);

/* kernels/v3/v3_tensorcore.cu:752-790 extended to the mask: the reference's
 * v3 is one kernel per head_dim, while each configuration here has a dense
 * and a causal instantiation with their own registers, spills and occupancy
 * (fa_query_fused and fa_query_fused_groups describe the dense one).
 * fa_query_fused_config reports the kernel fa_launch_attention_fused_groups
 * runs for (rows_per_block, kv_groups) with this mask;
 * fa_query_tensorcore_v3_shape reports the kernel
 * fa_launch_attention_tensorcore_v3 launches at this shape and mask on the
 * current device (its configuration as fa_tensorcore_v3_config names it).
 * An unsupported head_dim gives supported = 0 and status 0, as
 * fa_query_tensorcore_v3. */
int fa_query_fused_config(int head_dim, int rows_per_block, int kv_groups, int causal, fa_tiling_info* info);
int fa_query_tensorcore_v3_shape(int batch, int heads, int seq_len, int head_dim, int causal,
                                 fa_tiling_info* info);

/* No counterpart in the reference (whose v3 has one configuration): the
 * workgroup configuration fa_launch_attention_tensorcore_v3 runs at this
 * shape on the current device, as (query rows per workgroup, KV wave groups):
 * (64, 2), (64, 4), (128, 2) or (256, 1). FA_ERROR_UNSUPPORTED (both set to
 * 0) for an unsupported head_dim. fa_tensorcore_v3_rows_per_block returns the
 * rows alone (0 for an unsupported head_dim). */
int fa_tensorcore_v3_config(int batch, int heads, int seq_len, int head_dim, int causal,
                            int* rows_per_block, int* kv_groups);
int fa_tensorcore_v3_rows_per_block(int batch, int heads, int seq_len, int head_dim, int causal);

/* include/flash_attention.h:94, kernels/v3/v3_tensorcore.cu:752-790 — the
 * 128-row (two wave group) configuration, the one the reference's
 * single-configuration query corresponds to; fa_query_fused reports the
 * others and fa_tensorcore_v3_rows_per_block says which one a shape runs. */
int fa_query_tensorcore_v3(int head_dim, fa_tiling_info* info);

/* include/flash_attention.h:96, kernels/v3/v3_tensorcore.cu:795-818 — the
 * algorithmic HBM model of the fused kernel in the configuration and layout
 * the v3 entry runs at this shape: Q read and O written once, every K/V
 * tile counted once per workgroup that walks it. Contiguous row blocks walk
 * the tiles up to their last key (the reference's accounting); causal grids
 * of one round pair half blocks p and last - p, so a two-group workgroup
 * walks up to its later half block's last key and the list layout walks
 * both half blocks' tiles, the shared ones twice (at (2,8,2048,64) causal
 * 1056 tiles per slab against 544 for contiguous blocks). An upper bound on
 * HBM traffic: L2 reuse brings the measured figure to Q+K+V+O once. */
double fa_tensorcore_v3_hbm_bytes(int batch, int heads, int seq_len, int head_dim, int causal);

/* include/flash_attention.h:101-107 — the reference's v3b occupancy variant.
 * Here: the same MFMA arithmetic with 64 query rows per workgroup (twice the
 * workgroups, for shapes that leave CUs idle at 128 rows). */
int fa_tensorcore_v3b_supported(int head_dim);
int fa_launch_attention_tensorcore_v3b(const void* q, const void* k, const void* v, void* o,
                                       int batch, int heads, int seq_len, int head_dim,
                                       int causal, void* stream);
int fa_query_tensorcore_v3b(int head_dim, fa_tiling_info* info);
double fa_tensorcore_v3b_hbm_bytes(int batch, int heads, int seq_len, int head_dim, int causal);

/* Harness support (benchmarks/bench_flash_attention.cu:265-299): run
 * `warmup` untimed launches of kernel `which` (0 = unfused, 1 = v3 fused,
 * 2 = v3b fused, 3 = fused with 128 rows per workgroup whatever the shape,
 * 4 = fused with 256 rows per workgroup, 5 = fused with 64 rows and four
 * KV groups, 6 = fused with 128 rows and four KV groups: the list layout,
 * head_dim 64),
 * synchronise, then `iters` launches each bracketed by
 * hipEventRecord on `stream`; elapsed milliseconds go to samples_ms[iters].
 * Returns FA_ERROR_UNSUPPORTED for an unsupported head_dim and
 * hipErrorInvalidValue for a non-positive or non-finite sample. */
int fa_time_launches(int which, const void* q, const void* k, const void* v, void* o,
                     float* workspace, int batch, int heads, int seq_len, int head_dim,
                     int causal, int warmup, int iters, float* samples_ms, void* stream);

/* Throughput form: `iters` back-to-back launches between one pair of events;
 * total elapsed milliseconds in *total_ms. */
int fa_time_batch(int which, const void* q, const void* k, const void* v, void* o,
                  float* workspace, int batch, int heads, int seq_len, int head_dim,
                  int causal, int iters, float* total_ms, void* stream);

/* No counterpart in the reference (its numbers are quoted against a fixed
 * published peak only): a same-run calibration of the dense bf16 matrix
 * rate the device sustains. One untimed launch, then `launches` timed
 * launches (one hipEvent pair on `stream`) of a kernel with one 512-thread
 * workgroup per CU in which every wave (two per SIMD) issues
 * `mfma_per_wave` (>= 8; rounded down to a multiple of 8) back-to-back
 * v_mfma_f32_32x32x16_bf16 on four independent accumulators. `records` is a
 * device buffer of fa_mfma_peak_records_bytes() bytes (the kernel's per-
 * workgroup clock stamps). `operands` is NULL (hashed bf16 values in
 * [-1, -0.5] U [0.5, 1]) or a device pointer to 4096 bf16 values the MFMA
 * operands are drawn from (a workload's own Q and K, say): the clock the
 * device holds under this load depends on the data's switching power
 * (measured on MI355X: zeros 2.39 GHz, uniform[-1,1) 1.94 GHz, N(0, 3^2)
 * 1.76 GHz). Synchronises `stream`. *tflops: the rate over the timed
 * launches; *clock_ghz: the median shader clock of the last launch
 * (s_memtime ticks over s_memrealtime wall time). For bench.py's
 * roofline.sustained_peak: the published 2.5 PFLOP/s assumes 2.4 GHz, which
 * the device holds under full MFMA load only for low-activity data. */
size_t fa_mfma_peak_records_bytes(void);
int fa_mfma_peak(const void* operands, int mfma_per_wave, int launches, void* records, double* tflops,
                 double* clock_ghz, void* stream);

/* Library identification: "gfx950" and the build's kernel configuration. */
const char* fa_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
