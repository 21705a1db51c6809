// flash_attention_v0_profile.h — the reference's v0 stage-profiling interface
// (include/flash_attention_v0_profile.h:1-25 of RichterWang/cuda_fused_attention)
// with hipEvent_t / hipError_t / hipStream_t in place of the CUDA types.
#pragma once

#include "flash_attention.h"

namespace cuda_op_lab::flash_attention {

// Caller owns timing-enabled events and waits for pv_end before reading times.
// All events and launches use the same stream. Workspace matches v0.
struct V0ProfileEvents
{
    hipEvent_t qk_start;
    hipEvent_t qk_end;
    hipEvent_t softmax_end;
    hipEvent_t pv_end;
};

// Same preconditions as launch_attention_unfused. Returns event-record and
// launch errors; asynchronous errors surface on stream synchronisation. A null
// events pointer launches exactly the three kernels with no markers.
hipError_t launch_attention_unfused_profile(const __hip_bfloat16* q, const __hip_bfloat16* k,
                                            const __hip_bfloat16* v, __hip_bfloat16* o, float* workspace,
                                            const AttentionShape& shape, bool causal,
                                            const V0ProfileEvents* events = nullptr,
                                            hipStream_t stream = nullptr);

}  // namespace cuda_op_lab::flash_attention
