#pragma once
// wave:: prefix scans, reference-compatible API, wave64.
//
// Same names and return types as the reference's portable scans
// (research/wave-primitives/include/wave_primitives/wave_scan.hpp:38-167):
// scan_inclusive_sum / _max / _min and scan_exclusive_sum for any arithmetic T and for
// __half / bf16 (fp32 accumulation, result rounded back to the input type). Built on
// the zero-LDS DPP + permlane scan of detail/xlane.hpp instead of __shfl_up.
#include "detail/xlane.hpp"
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <hip/hip_bfloat16.h>

namespace wave {

template <typename T> __device__ __forceinline__ T scan_inclusive_sum(T v) { return xlane::scan_inclusive(v, xlane::Sum{}); }
template <typename T> __device__ __forceinline__ T scan_inclusive_max(T v) { return xlane::scan_inclusive(v, xlane::Max{}); }
template <typename T> __device__ __forceinline__ T scan_inclusive_min(T v) { return xlane::scan_inclusive(v, xlane::Min{}); }
template <typename T> __device__ __forceinline__ T scan_exclusive_sum(T v) { return xlane::scan_exclusive(v, xlane::Sum{}); }

#define WAVE_HALF_SCAN(NAME)                                                                  \
    __device__ __forceinline__ __half NAME(__half v) { return __float2half(NAME(__half2float(v))); } \
    __device__ __forceinline__ __hip_bfloat16 NAME(__hip_bfloat16 v) {                        \
        return __float2bfloat16(NAME(__bfloat162float(v)));                                   \
    }                                                                                         \
    __device__ __forceinline__ hip_bfloat16 NAME(hip_bfloat16 v) { return hip_bfloat16(NAME(float(v))); }
WAVE_HALF_SCAN(scan_inclusive_sum)
WAVE_HALF_SCAN(scan_inclusive_max)
WAVE_HALF_SCAN(scan_inclusive_min)
WAVE_HALF_SCAN(scan_exclusive_sum)
#undef WAVE_HALF_SCAN

}  // namespace wave
