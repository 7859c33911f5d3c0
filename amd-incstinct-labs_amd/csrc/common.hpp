// Shared host/device helpers of libcdna4_attn.so (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>
#include "cdna4_attn.h"

namespace cdna4 {

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

// ---- element types ----------------------------------------------------------
__device__ __forceinline__ float f32_from_bits(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- host side ------------------------------------------------------------------
// 0 when the current device is gfx950, else CDNA4_ERR_INVALID_DEVICE_FUNCTION or the
// runtime error. The answer is cached per device ordinal.
int check_device();

// Compute units of the current device (cached per device ordinal; 256 if the query fails).
int device_cus();

inline int launch_status() {
    hipError_t e = hipGetLastError();
    return (int)e;
}

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace cdna4
