// Prompt-path GEMM of the small-LLM runtime (gfx950): Y[M][N] (+)= X[M][K] W[N][K]^T with fp16
// X and W (both row-major, K contiguous), fp32 accumulation, fp32 or fp16 Y.
//
// Reference behaviour restated: the reference runs these products through rocBLAS gemm_ex
// (cdna3-prims/include/cdna3/runtime/rocblas_gemm.hpp:8-20; forward.hpp:70-131), Y = X W^T with W
// the [out][in] weight as the model files hold it, beta 0 (Q|K|V, gate|up) or 1 (the O and down
// projections added into the fp32 residual).
//
// MI355X design: at prompt lengths of a few hundred tokens these GEMMs are small (0.6-4.8 GFLOP)
// and rocBLAS's choice for them ran at ~180 TFLOP/s. Here a workgroup of four waves computes a
// BM x BN tile of Y^T = W X^T on v_mfma_f32_16x16x32_f16: W rows are the A operand and X rows the
// B operand, so a lane's accumulator holds four consecutive columns n of one row m and leaves as
// one 16-byte (fp32) or 8-byte (fp16) store. Each 64-wide K step of both operand tiles is copied
// HBM -> registers -> LDS (16-byte loads, eight threads per 128-byte row), double-buffered: the
// next step's loads are in flight while the MFMAs consume the current one. Rows past M or N read
// the last valid row (their results are not stored). The tile is the largest of 128 x 128,
// 64 x 128 and 64 x 64 (m x n) whose grid still covers the CUs.
#include "common.hpp"

namespace cdna4 {
namespace {

typedef _Float16 gf16x8 __attribute__((ext_vector_type(8)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 gf16x4 __attribute__((ext_vector_type(4)));

constexpr int kKMul = 64;   // K must be a multiple of this (the smallest stage)

// KT: K per LDS stage (KT / 32 MFMA K steps); rows padded by 8 halves against bank conflicts.
template <int BM, int BN, int KT, bool kF32Out, bool kAccum>
__global__ __launch_bounds__(256) void gemm_f16_nt(const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                                                   void* __restrict__ Y, int M, int N, int K, int ldy) {
    constexpr int FN = BN / 32, FM = BM / 32;   // 16-row MFMA blocks per wave (n, m)
    constexpr int kLdsRow = KT + 8;
    constexpr int kRowChunks = KT / 8;          // 16-byte chunks per row and stage
    constexpr int CX = BM * kRowChunks / 256;   // 16-byte chunks per thread and stage (X)
    constexpr int CW = BN * kRowChunks / 256;   // (W)
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][BN * kLdsRow];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = (int)blockIdx.x * BM, n0 = (int)blockIdx.y * BN;

    // Loader: chunk c = tid + 256 j of a stage is row c / kRowChunks, 16-byte column c % kRowChunks.
    u32x4 rx[CX], rw[CW];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < CX; ++j) {
            const int c = tid + 256 * j, r = min(m0 + c / kRowChunks, M - 1);
            rx[j] = *(const u32x4*)(X + (size_t)r * K + k0 + (c % kRowChunks) * 8);
        }
#pragma unroll
        for (int j = 0; j < CW; ++j) {
            const int c = tid + 256 * j, r = min(n0 + c / kRowChunks, N - 1);
            rw[j] = *(const u32x4*)(W + (size_t)r * K + k0 + (c % kRowChunks) * 8);
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < CX; ++j) {
            const int c = tid + 256 * j;
            *(u32x4*)(&xs[st][(c / kRowChunks) * kLdsRow + (c % kRowChunks) * 8]) = rx[j];
        }
#pragma unroll
        for (int j = 0; j < CW; ++j) {
            const int c = tid + 256 * j;
            *(u32x4*)(&ws[st][(c / kRowChunks) * kLdsRow + (c % kRowChunks) * 8]) = rw[j];
        }
    };

    gf32x4 acc[FN][FM];
#pragma unroll
    for (int a = 0; a < FN; ++a)
#pragma unroll
        for (int b = 0; b < FM; ++b) acc[a][b] = gf32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = K / KT;
    gload(0);
    lstore(0);
    __syncthreads();
    const int r16 = lane & 15, g8 = (lane >> 4) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * KT);
#pragma unroll
        for (int ks = 0; ks < KT; ks += 32) {
            u32x4 a[FN], b[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i)
                a[i] = *(const u32x4*)(&ws[st][(wn * (BN / 2) + i * 16 + r16) * kLdsRow + ks + g8]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                b[i] = *(const u32x4*)(&xs[st][(wm * (BM / 2) + i * 16 + r16) * kLdsRow + ks + g8]);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(gf16x8, a[i]),
                                                                       __builtin_bit_cast(gf16x8, b[j]), acc[i][j], 0,
                                                                       0, 0);
        }
        if (kt + 1 < nk) lstore(st ^ 1);
        __syncthreads();
    }

    // acc[i][j] lane l: Y[m][n .. n + 3], m = row r16 of X block j, n = 4 (l / 16) of W block i.
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * (BM / 2) + j * 16 + r16;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int n = n0 + wn * (BN / 2) + i * 16 + (lane >> 4) * 4;
            if (n >= N) continue;
            gf32x4 v = acc[i][j];
            if constexpr (kF32Out) {
                float* y = (float*)Y + (size_t)m * ldy + n;
                if constexpr (kAccum) v += *(const gf32x4*)y;
                *(gf32x4*)y = v;
            } else {
                _Float16* y = (_Float16*)Y + (size_t)m * ldy + n;
                if constexpr (kAccum) {
                    const gf16x4 o = *(const gf16x4*)y;
                    v += gf32x4{(float)o[0], (float)o[1], (float)o[2], (float)o[3]};
                }
                *(gf16x4*)y = gf16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            }
        }
    }
}

template <int BM, int BN, int KT>
int gemm_launch(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, bool accum, int M, int N, int K, int ldy,
                hipStream_t s) {
    const dim3 grid((unsigned)ceil_div((size_t)M, BM), (unsigned)ceil_div((size_t)N, BN));
    if (y_f32) {
        if (accum) gemm_f16_nt<BM, BN, KT, true, true><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy);
        else gemm_f16_nt<BM, BN, KT, true, false><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy);
    } else {
        if (accum) gemm_f16_nt<BM, BN, KT, false, true><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy);
        else gemm_f16_nt<BM, BN, KT, false, false><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy);
    }
    return launch_status();
}

}  // namespace

// Returns -1, launching nothing, for a shape this kernel does not take (K not a multiple of 64,
// N or ldy not a multiple of 4, X / W not 16-byte or Y not 16- (fp32) / 8-byte (fp16) aligned);
// the caller then uses rocBLAS. Otherwise 0 or the launch's error.
int llm_gemm_f16(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, bool accum, int M, int N, int K, int ldy,
                 hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0 || K % kKMul || N % 4 || ldy % 4 || ldy < N) return -1;
    if (((uintptr_t)X | (uintptr_t)W) % 16 || (uintptr_t)Y % (y_f32 ? 16 : 8)) return -1;
    const size_t cus = (size_t)(device_cus() > 0 ? device_cus() : 256);
    auto tiles = [&](size_t bm, size_t bn) { return ceil_div((size_t)M, bm) * ceil_div((size_t)N, bn); };
    // the deepest stage (fewest exposed memory round trips) that divides K and fits the LDS
    if (tiles(128, 128) >= cus) {
        if (K % 128 == 0) return gemm_launch<128, 128, 128>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
        return gemm_launch<128, 128, 64>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
    }
    if (tiles(64, 128) >= cus) {
        if (K % 128 == 0) return gemm_launch<64, 128, 128>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
        return gemm_launch<64, 128, 64>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
    }
    if (K % 256 == 0) return gemm_launch<64, 64, 256>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
    if (K % 128 == 0) return gemm_launch<64, 64, 128>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
    return gemm_launch<64, 64, 64>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
}

}  // namespace cdna4

extern "C" int cdna4_gemm_f16_nt(const void* X, const void* W, void* Y, int y_f32, int accum, int M, int N, int K,
                                 int ldy, cdna4_stream_t stream) {
    if (M < 0 || N < 0 || K < 0 || (y_f32 != 0 && y_f32 != 1) || (accum != 0 && accum != 1))
        return CDNA4_ERR_INVALID_VALUE;
    if (M == 0 || N == 0) return 0;
    if (!X || !W || !Y) return CDNA4_ERR_INVALID_VALUE;
    if (int e = cdna4::check_device()) return e;
    const int e = cdna4::llm_gemm_f16((const uint16_t*)X, (const uint16_t*)W, Y, y_f32 == 1, accum == 1, M, N, K, ldy,
                                      (hipStream_t)stream);
    return e == -1 ? CDNA4_ERR_INVALID_VALUE : e;
}
