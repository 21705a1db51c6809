// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <tuple>
#include <type_traits>
#include <utility>

namespace fa {

// Launches `kernel` on `stream` through hipLaunchKernel and returns the
// runtime's status for this launch alone (no hipGetLastError, so an earlier,
// unrelated error is neither reported here nor cleared; a failed launch
// stays in HIP's own last-error state as well, where a caller's
// hipGetLastError finds it). Arguments are converted to the kernel's
// parameter types first.
template <typename... Params, typename... Args>
hipError_t launch_kernel(void (*kernel)(Params...), dim3 grid, dim3 block, hipStream_t stream, Args&&... args)
{
    static_assert(sizeof...(Params) == sizeof...(Args) && sizeof...(Params) > 0, "kernel argument count");
    std::tuple<std::decay_t<Params>...> values{static_cast<std::decay_t<Params>>(std::forward<Args>(args))...};
    return std::apply(
        [&](auto&... v) {
            void* ptrs[] = {static_cast<void*>(&v)...};
            return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, 0, stream);
        },
        values);
}

// Records a non-success status of a C-ABI call in the calling thread's
// last-error slot (read by fa_get_last_error / fa_peek_at_last_error) and
// returns it unchanged. FA_ERROR_UNSUPPORTED (an unsupported head_dim, which
// the reference's launchers skip silently) is not recorded. Defined in
// fa_api.cpp.
int record_status(int status);

// bf16 is carried as raw 16-bit patterns in memory (uint16_t); conversions
// below are exact (bf16 -> f32) or IEEE round-to-nearest-even (f32 -> bf16,
// lowered to v_cvt_pk_bf16_f32 on gfx950).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16)
{
    return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t word) { return __uint_as_float(word & 0xffff0000u); }

// Two floats -> packed bf16x2 word (low half = a), RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b)
{
    bf16x2 v;
    v[0] = static_cast<__bf16>(a);
    v[1] = static_cast<__bf16>(b);
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t float_to_bf16_bits(float a)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(a));
}

// wave64 reductions (butterfly over all 64 lanes)
__device__ __forceinline__ float wave_max(float x)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) x = fmaxf(x, __shfl_xor(x, offset, 64));
    return x;
}

__device__ __forceinline__ float wave_sum(float x)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) x += __shfl_xor(x, offset, 64);
    return x;
}

constexpr float kLog2e = 1.4426950408889634f;

// Map a linear workgroup id onto the hardware's round-robin dispatch over the
// 8 XCDs of an MI355X so that logically consecutive workgroups (which share a
// (batch, head) slab's K and V) run on the same XCD and share its L2. A
// bijection on [0, total) whenever total is a multiple of 8; identity
// otherwise.
__device__ __forceinline__ int xcd_remap(int linear, int total)
{
    constexpr int kXcds = 8;
    if (total % kXcds != 0) return linear;
    const int per_xcd = total / kXcds;
    return (linear % kXcds) * per_xcd + linear / kXcds;
}

}  // namespace fa
