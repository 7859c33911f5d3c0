#pragma once
// cdna3::ex — the asynchronous-copy + matrix-core tile loop building block (gfx950).
//
// Same name and arguments as the reference's composition example
// (cdna3-prims/examples/async_tiled_gemm.hpp:52-60): one 16x16 fp16 tile product
// C = A B with fp32 accumulation, A, B, C row-major with leading dimensions ldA, ldB, ldC, read
// and written by one wave (lane = 0..63) through the verified 16x16x16 lane mapping.
//
// The tile-loop order that example documents holds on gfx950 too: issue the asynchronous copy
// of tile t + 1 (dme::copy_tile_16B / prefetch_tile2d_fp16, 16 bytes per lane) before computing
// tile t, and wait for it (dme::wait, then a barrier when other waves read it) only after that
// compute. The attention kernels of libcdna4_attn.so use exactly this order with double buffers.
// mma_tile_accumulate_k32 is the CDNA4 double-rate form (16x16x32, f16 or bf16): the same tile
// product over a K of 32 in one instruction.
#include "../cdna3.hpp"

namespace cdna3 {
namespace ex {

__device__ __forceinline__ void mma_tile_accumulate(const __half* A_lds, const __half* B_lds, float* C_lds, int lane,
                                                    int ldA, int ldB, int ldC) {
    const mfma::fp16x4 a = mfma::load_A(A_lds, lane, ldA);
    const mfma::fp16x4 b = mfma::load_B(B_lds, lane, ldB);
    mfma::f32x4 c = {0.f, 0.f, 0.f, 0.f};
    c = mfma::mma(a, b, c);
    mfma::store_C(C_lds, c, lane, ldC);
}

// C[16 x 16] = A[16 x 32] B[32 x 16] on v_mfma_f32_16x16x32_{f16,bf16}; T = _Float16 or __bf16.
template <typename T>
__device__ __forceinline__ void mma_tile_accumulate_k32(const T* A_lds, const T* B_lds, float* C_lds, int lane,
                                                        int ldA, int ldB, int ldC) {
    using V = typename std::conditional<std::is_same<T, __bf16>::value, cdna4::mfma::bf16x8, cdna4::mfma::f16x8>::type;
    const V a = cdna4::mfma::load_A_16x16x32<V>(A_lds, lane, ldA);
    const V b = cdna4::mfma::load_B_16x16x32<V>(B_lds, lane, ldB);
    cdna4::mfma::f32x4 c = {0.f, 0.f, 0.f, 0.f};
    c = cdna4::mfma::mma_16x16x32(a, b, c);
    cdna4::mfma::store_C_16x16x32(C_lds, c, lane, ldC);
}

}  // namespace ex
}  // namespace cdna3
