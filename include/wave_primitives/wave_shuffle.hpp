#pragma once
// wave:: lane id and shuffles, wave64.
//
// Names and semantics follow the reference's portable shuffle API
// (research/wave-primitives/include/wave_primitives/wave_shuffle.hpp:24-117): lane_id,
// shfl, shfl_down, shfl_up, shfl_xor, with __half / bf16 overloads that move the value
// as fp32. Arbitrary-lane shuffles are routed through ds_bpermute by the hardware;
// code that needs zero LDS instructions uses the wave::dpp reductions and scans.
#include "detail/config.hpp"
#include "detail/xlane.hpp"
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <hip/hip_bfloat16.h>

namespace wave {

__device__ __forceinline__ unsigned int lane_id() { return xlane::lane(); }

template <typename T>
__device__ __forceinline__ T shfl(T val, int src_lane, int width = kWaveSize) { return __shfl(val, src_lane, width); }
template <typename T>
__device__ __forceinline__ T shfl_down(T val, unsigned int delta, int width = kWaveSize) { return __shfl_down(val, delta, width); }
template <typename T>
__device__ __forceinline__ T shfl_up(T val, unsigned int delta, int width = kWaveSize) { return __shfl_up(val, delta, width); }
template <typename T>
__device__ __forceinline__ T shfl_xor(T val, int lane_mask, int width = kWaveSize) { return __shfl_xor(val, lane_mask, width); }

#define WAVE_HALF_SHFL(NAME, ARGT)                                                          \
    __device__ __forceinline__ __half NAME(__half v, ARGT a, int width = kWaveSize) {       \
        return __float2half(NAME(__half2float(v), a, width));                               \
    }                                                                                       \
    __device__ __forceinline__ __hip_bfloat16 NAME(__hip_bfloat16 v, ARGT a, int width = kWaveSize) { \
        return __float2bfloat16(NAME(__bfloat162float(v), a, width));                       \
    }                                                                                       \
    __device__ __forceinline__ hip_bfloat16 NAME(hip_bfloat16 v, ARGT a, int width = kWaveSize) { \
        return hip_bfloat16(NAME(float(v), a, width));                                      \
    }
WAVE_HALF_SHFL(shfl, int)
WAVE_HALF_SHFL(shfl_down, unsigned int)
WAVE_HALF_SHFL(shfl_up, unsigned int)
WAVE_HALF_SHFL(shfl_xor, int)
#undef WAVE_HALF_SHFL

}  // namespace wave
