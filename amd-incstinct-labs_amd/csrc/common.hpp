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

// Rotate-half RoPE of one (d, d + D/2) pair of fp16 values with the pair's cos/sin entries
// (shared by the fused RoPE + append kernel and the prompt GEMM's Q|K|V epilogue, so both round
// alike).
__device__ __forceinline__ void rope_pair(uint32_t a_bits, uint32_t b_bits, float c_lo, float s_lo, float c_hi,
                                          float s_hi, uint32_t& lo, uint32_t& hi) {
    const float a = f16_bits_to_f32(a_bits), b = f16_bits_to_f32(b_bits);
    lo = f32_to_f16_bits(a * c_lo + (-b) * s_lo);
    hi = f32_to_f16_bits(b * c_hi + a * s_hi);
}

// Destinations of the prompt GEMM's Q|K|V epilogue (gemm.hip, llm_gemm_qkv_rope): queries
// head-major [QD / D][T][D], keys and values into the caches [heads][max_seq][D] at rows
// pos0 .. pos0 + T - 1, cos/sin tables [position][D].
struct QkvOut {
    uint16_t *q_out, *Kc, *Vc;
    const float *cosv, *sinv;
    int QD, KVD, D, T, pos0, max_seq;
};

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
