#pragma once
// cdna3/mfma.hpp — typed matrix-core accessors with verified wave64 lane mappings (gfx950).
//
// cdna3::mfma:: keeps the reference's 16x16x16 f16 API unchanged (cdna3-prims/include/
// cdna3/mfma.hpp:27-91: M, N, K, FRAGS, fp16x4, f32x4, to_fp16, mma, load_A, load_B,
// store_C, store_C_fp16); v_mfma_f32_16x16x16_f16 is still a gfx950 instruction with the
// same lane mapping:
//   A: lane L, frag f -> A[L%16][(L/16)*4+f];  B: B[(L/16)*4+f][L%16];  C: C[(L/16)*4+f][L%16]
//
// cdna4::mfma:: adds the CDNA4 double-rate tiles, lane mappings checked on an MI355X with an
// exact small-integer GEMM against a host matmul:
//   16x16x32 (f16, bf16): A lane L, e in 0..7 -> A[L%16][(L/16)*8+e]
//                         B              -> B[(L/16)*8+e][L%16]
//                         C, e in 0..3   -> C[(L/16)*4+e][L%16]
//   32x32x16 (f16, bf16): A -> A[L%32][(L/32)*8+e];  B -> B[(L/32)*8+e][L%32]
//                         C, e in 0..15 -> C[(e/4)*8 + (L/32)*4 + e%4][L%32]
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

namespace cdna3 {
namespace mfma {

static constexpr int M = 16;
static constexpr int N = 16;
static constexpr int K = 16;
static constexpr int FRAGS = 4;   // elements each lane holds of A, B, and C

using fp16x4 = __attribute__((ext_vector_type(4))) __fp16;
using f32x4 = __attribute__((ext_vector_type(4))) float;

__device__ __forceinline__ __fp16 to_fp16(__half h) { return __builtin_bit_cast(__fp16, h); }

__device__ __forceinline__ f32x4 mma(fp16x4 a, fp16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ fp16x4 load_A(const __half* A_tile, int lane, int ldA = K) {
    fp16x4 a;
    const int row = lane % 16, k0 = (lane / 16) * 4;
#pragma unroll
    for (int f = 0; f < 4; ++f) a[f] = to_fp16(A_tile[row * ldA + k0 + f]);
    return a;
}

__device__ __forceinline__ fp16x4 load_B(const __half* B_tile, int lane, int ldB = N) {
    fp16x4 b;
    const int col = lane % 16, k0 = (lane / 16) * 4;
#pragma unroll
    for (int f = 0; f < 4; ++f) b[f] = to_fp16(B_tile[(k0 + f) * ldB + col]);
    return b;
}

__device__ __forceinline__ void store_C(float* C_tile, f32x4 c, int lane, int ldC = N) {
    const int col = lane % 16, r0 = (lane / 16) * 4;
#pragma unroll
    for (int f = 0; f < 4; ++f) C_tile[(r0 + f) * ldC + col] = c[f];
}

__device__ __forceinline__ void store_C_fp16(__half* C_tile, f32x4 c, int lane, int ldC = N) {
    const int col = lane % 16, r0 = (lane / 16) * 4;
#pragma unroll
    for (int f = 0; f < 4; ++f) C_tile[(r0 + f) * ldC + col] = __float2half(c[f]);
}

}  // namespace mfma
}  // namespace cdna3

namespace cdna4 {
namespace mfma {

using f16x8 = __attribute__((ext_vector_type(8))) _Float16;
using bf16x8 = __attribute__((ext_vector_type(8))) __bf16;
using f32x4 = __attribute__((ext_vector_type(4))) float;
using f32x16 = __attribute__((ext_vector_type(16))) float;

// ---- 16x16x32 ---------------------------------------------------------------------------
struct K32 {
    static constexpr int M = 16, N = 16, K = 32, FRAGS_AB = 8, FRAGS_C = 4;
};

__device__ __forceinline__ f32x4 mma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Row-major tiles of 16-bit elements (T = _Float16 or __bf16).
template <typename V, typename T>
__device__ __forceinline__ V load_A_16x16x32(const T* A, int lane, int ldA = 32) {
    V a;
    const int row = lane % 16, k0 = (lane / 16) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = A[row * ldA + k0 + e];
    return a;
}
template <typename V, typename T>
__device__ __forceinline__ V load_B_16x16x32(const T* B, int lane, int ldB = 16) {
    V b;
    const int col = lane % 16, k0 = (lane / 16) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = B[(k0 + e) * ldB + col];
    return b;
}
__device__ __forceinline__ void store_C_16x16x32(float* C, f32x4 c, int lane, int ldC = 16) {
    const int col = lane % 16, r0 = (lane / 16) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) C[(r0 + e) * ldC + col] = c[e];
}

// ---- 32x32x16 ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <typename V, typename T>
__device__ __forceinline__ V load_A_32x32x16(const T* A, int lane, int ldA = 16) {
    V a;
    const int row = lane % 32, k0 = (lane / 32) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = A[row * ldA + k0 + e];
    return a;
}
template <typename V, typename T>
__device__ __forceinline__ V load_B_32x32x16(const T* B, int lane, int ldB = 32) {
    V b;
    const int col = lane % 32, k0 = (lane / 32) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = B[(k0 + e) * ldB + col];
    return b;
}
__device__ __forceinline__ void store_C_32x32x16(float* C, f32x16 c, int lane, int ldC = 32) {
    const int col = lane % 32, r0 = (lane / 32) * 4;
#pragma unroll
    for (int e = 0; e < 16; ++e) C[((e / 4) * 8 + r0 + e % 4) * ldC + col] = c[e];
}

// ---- 16x16x4 fp32 ------------------------------------------------------------------------
// fp32 products and accumulation; lane L holds A[L % 16][L / 16], B[L / 16][L % 16] and
// C[4 (L / 16) + i][L % 16] (the 16x16x32 C layout).
__device__ __forceinline__ f32x4 mma_16x16x4f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float load_A_16x16x4f32(const float* A, int lane, int ldA = 4) {
    return A[(lane % 16) * ldA + lane / 16];
}
__device__ __forceinline__ float load_B_16x16x4f32(const float* B, int lane, int ldB = 16) {
    return B[(lane / 16) * ldB + lane % 16];
}
__device__ __forceinline__ void store_C_16x16x4f32(float* C, f32x4 c, int lane, int ldC = 16) {
    store_C_16x16x32(C, c, lane, ldC);
}

}  // namespace mfma
}  // namespace cdna4
