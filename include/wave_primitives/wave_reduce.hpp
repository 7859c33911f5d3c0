#pragma once
// wave:: reductions, reference-compatible API, wave64.
//
// Same names and return types as the reference's portable reductions
// (research/wave-primitives/include/wave_primitives/wave_reduce.hpp:38-141):
// reduce_sum / reduce_max / reduce_min for any arithmetic T and for __half / bf16
// (fp32 accumulation, result rounded back to the input type), and reduce_and /
// reduce_or for integers. The reference built these on __shfl_down (ds_bpermute);
// here they are the zero-LDS butterfly of detail/xlane.hpp, so the result is valid
// on every lane (the reference guaranteed lane 0 only).
#include "detail/xlane.hpp"
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <hip/hip_bfloat16.h>

namespace wave {

template <typename T> __device__ __forceinline__ T reduce_sum(T v) { return xlane::allreduce(v, xlane::Sum{}); }
template <typename T> __device__ __forceinline__ T reduce_max(T v) { return xlane::allreduce(v, xlane::Max{}); }
template <typename T> __device__ __forceinline__ T reduce_min(T v) { return xlane::allreduce(v, xlane::Min{}); }

__device__ __forceinline__ __half reduce_sum(__half v) { return __float2half(reduce_sum(__half2float(v))); }
__device__ __forceinline__ __half reduce_max(__half v) { return __float2half(reduce_max(__half2float(v))); }
__device__ __forceinline__ __half reduce_min(__half v) { return __float2half(reduce_min(__half2float(v))); }
__device__ __forceinline__ __hip_bfloat16 reduce_sum(__hip_bfloat16 v) { return __float2bfloat16(reduce_sum(__bfloat162float(v))); }
__device__ __forceinline__ __hip_bfloat16 reduce_max(__hip_bfloat16 v) { return __float2bfloat16(reduce_max(__bfloat162float(v))); }
__device__ __forceinline__ __hip_bfloat16 reduce_min(__hip_bfloat16 v) { return __float2bfloat16(reduce_min(__bfloat162float(v))); }
// hip_bfloat16 (the struct type of <hip/hip_bfloat16.h>) is the type the reference's
// overloads take (wave_reduce.hpp:57-63).
__device__ __forceinline__ hip_bfloat16 reduce_sum(hip_bfloat16 v) { return hip_bfloat16(reduce_sum(float(v))); }
__device__ __forceinline__ hip_bfloat16 reduce_max(hip_bfloat16 v) { return hip_bfloat16(reduce_max(float(v))); }
__device__ __forceinline__ hip_bfloat16 reduce_min(hip_bfloat16 v) { return hip_bfloat16(reduce_min(float(v))); }

template <typename T>
__device__ __forceinline__ T reduce_and(T v) {
    static_assert(std::is_integral<T>::value, "reduce_and requires an integer type");
    return xlane::allreduce(v, xlane::And{});
}
template <typename T>
__device__ __forceinline__ T reduce_or(T v) {
    static_assert(std::is_integral<T>::value, "reduce_or requires an integer type");
    return xlane::allreduce(v, xlane::Or{});
}

}  // namespace wave
