// Test hooks (tests only, not part of libcdna4_attn.so): run the header-only device templates
// of include/ (wave::dpp, wave::, cdna3::mfma, cdna4::mfma, dme::, cdna3::ex) on whole waves so
// that pytest can check them lane by lane against closed forms and the CPU oracle.
#include <hip/hip_runtime.h>
#include <cdna3/cdna3.hpp>
#include <cdna3/examples/fused_softmax.hpp>
#include <cdna3/examples/async_tiled_gemm.hpp>
#include <cdna3/runtime/forward.hpp>
#include <stdint.h>

namespace {

enum Kind {
    kDppSum = 0, kDppMax, kDppMin, kDppSumBcast, kDppScanSum, kDppScanMax, kDppScanMin, kDppScanExSum,
    kDppBcast63, kPortSum, kPortScanSum, kPortScanExSum, kPortAnd, kPortOr, kDppScanExMax, kSoftmaxLane,
    kPortMax, kPortMin, kDppMoveShr1, kDppStep1, kDppStep4, kDppStep1248, kNumKinds
};

template <typename In>
__device__ float widen(In v) {
    if constexpr (std::is_same<In, __half>::value) return __half2float(v);
    else return __bfloat162float(v);
}

// 32/64-bit element types: every kind except the fp16/bf16-only paths.
template <typename T>
__global__ void wave_kernel(int kind, const T* in, T* out) {
    const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
    const T x = in[i];
    T r = x;
    switch (kind) {
        case kDppSum: r = wave::dpp::reduce_sum(x); break;
        case kDppMax: r = wave::dpp::reduce_max(x); break;
        case kDppMin: r = wave::dpp::reduce_min(x); break;
        case kDppSumBcast: r = wave::dpp::reduce_sum_bcast(x); break;
        case kDppScanSum: r = wave::dpp::scan_inclusive_sum(x); break;
        case kDppScanMax: r = wave::dpp::scan_inclusive_max(x); break;
        case kDppScanMin: r = wave::dpp::scan_inclusive_min(x); break;
        case kDppScanExSum: r = wave::dpp::scan_exclusive_sum(x); break;
        case kDppBcast63: r = wave::dpp::bcast_lane63(x); break;
        case kPortSum: r = wave::reduce_sum(x); break;
        case kPortScanSum: r = wave::scan_inclusive_sum(x); break;
        case kPortScanExSum: r = wave::scan_exclusive_sum(x); break;
        case kPortAnd: if constexpr (std::is_integral<T>::value) r = wave::reduce_and(x); break;
        case kPortOr: if constexpr (std::is_integral<T>::value) r = wave::reduce_or(x); break;
        case kDppScanExMax: r = wave::dpp::scan_exclusive(x, wave::dpp::ScanMax{}); break;
        case kSoftmaxLane: if constexpr (std::is_same<T, float>::value) r = cdna3::ex::row_softmax_lane(x); break;
        case kPortMax: r = wave::reduce_max(x); break;
        case kPortMin: r = wave::reduce_min(x); break;
        case kDppMoveShr1: r = wave::dpp::dpp_move<0x111>(x, T(-7)); break;   // row_shr:1, row starts read -7
        case kDppStep1: r = wave::dpp::scan_dpp_step<1>(x, wave::dpp::ScanSum{}, T(0)); break;
        case kDppStep4: r = wave::dpp::scan_dpp_step<4>(x, wave::dpp::ScanMax{}, wave::dpp::scan_id_max<T>()); break;
        case kDppStep1248: {   // the four in-row steps: inclusive prefix within each 16-lane row
            const wave::dpp::ScanSum op{};
            r = wave::dpp::scan_dpp_step<1>(x, op, T(0));
            r = wave::dpp::scan_dpp_step<2>(r, op, T(0));
            r = wave::dpp::scan_dpp_step<4>(r, op, T(0));
            r = wave::dpp::scan_dpp_step<8>(r, op, T(0));
            break;
        }
        default: break;
    }
    out[i] = r;
}

// fp16 / bf16 inputs: wave::dpp forms accumulate in fp32 and return float; the portable
// wave:: forms round back to the input type (returned here widened to float).
template <typename In>
__global__ void wave_kernel_half(int kind, const In* in, float* out) {
    const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
    const In x = in[i];
    float r = 0.f;
    switch (kind) {
        case kDppSum: r = wave::dpp::reduce_sum(x); break;
        case kDppMax: r = wave::dpp::reduce_max(x); break;
        case kDppMin: r = wave::dpp::reduce_min(x); break;
        case kDppSumBcast: r = wave::dpp::reduce_sum_bcast(x); break;
        case kDppScanSum: r = wave::dpp::scan_inclusive_sum(x); break;
        case kDppScanMax: r = wave::dpp::scan_inclusive_max(x); break;
        case kDppScanMin: r = wave::dpp::scan_inclusive_min(x); break;
        case kDppScanExSum: r = wave::dpp::scan_exclusive_sum(x); break;
        case kPortSum: r = widen(wave::reduce_sum(x)); break;
        case kPortScanSum: r = widen(wave::scan_inclusive_sum(x)); break;
        case kPortScanExSum: r = widen(wave::scan_exclusive_sum(x)); break;
        case kPortMax: r = widen(wave::reduce_max(x)); break;
        case kPortMin: r = widen(wave::reduce_min(x)); break;
        default: r = widen(x); break;
    }
    out[i] = r;
}

// Ballot family on predicate (in[i] != 0): out = {ballot, popcount, any, all, lane_mask_lt}.
__global__ void ballot_kernel(const int32_t* in, uint64_t* out) {
    const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
    const int p = in[i] != 0;
    const size_t o = i * 5;
    out[o + 0] = wave::ballot(p);
    out[o + 1] = (uint64_t)wave::popcount(p);
    out[o + 2] = (uint64_t)wave::any(p);
    out[o + 3] = (uint64_t)wave::all(p);
    out[o + 4] = wave::lane_mask_lt();
}

// cdna3::mfma 16x16x16 f16 through the reference API (row-major A, B; C = A B).
__global__ void mfma16_kernel(const __half* A, const __half* B, float* C) {
    const int lane = threadIdx.x;
    cdna3::mfma::f32x4 c = {0.f, 0.f, 0.f, 0.f};
    c = cdna3::mfma::mma(cdna3::mfma::load_A(A, lane), cdna3::mfma::load_B(B, lane), c);
    cdna3::mfma::store_C(C, c, lane);
}

template <typename V, typename T>
__global__ void mfma16x32_kernel(const T* A, const T* B, float* C) {
    const int lane = threadIdx.x;
    cdna4::mfma::f32x4 c = {0.f, 0.f, 0.f, 0.f};
    c = cdna4::mfma::mma_16x16x32(cdna4::mfma::load_A_16x16x32<V>(A, lane), cdna4::mfma::load_B_16x16x32<V>(B, lane), c);
    cdna4::mfma::store_C_16x16x32(C, c, lane);
}

template <typename V, typename T>
__global__ void mfma32x16_kernel(const T* A, const T* B, float* C) {
    const int lane = threadIdx.x;
    cdna4::mfma::f32x16 c = {};
    c = cdna4::mfma::mma_32x32x16(cdna4::mfma::load_A_32x32x16<V>(A, lane), cdna4::mfma::load_B_32x32x16<V>(B, lane), c);
    cdna4::mfma::store_C_32x32x16(C, c, lane);
}

// dme: copy 4096 bytes with 16-byte lanes, 256 floats with 4-byte lanes, and a strided
// 16 x 64 fp16 tile (row stride 96 elements), each into LDS and back out.
__global__ void dme_kernel(const uint8_t* src, uint8_t* dst, const float* fsrc, float* fdst, const __half* hsrc,
                           __half* hdst) {
    __shared__ __attribute__((aligned(16))) uint8_t lds8[4096];
    __shared__ __attribute__((aligned(16))) float ldsf[256];
    __shared__ __attribute__((aligned(16))) __half ldsh[16 * 64];
    dme::copy_tile_16B<4096>(src, lds8);
    dme::copy_tile_1d<float, 256>(fsrc, ldsf);
    dme::prefetch_tile2d_strided_fp16<16, 64>(hsrc, ldsh, 96, threadIdx.x, 64);
    dme::wait();
    __syncthreads();
    for (int i = threadIdx.x; i < 4096; i += 64) dst[i] = lds8[i];
    for (int i = threadIdx.x; i < 256; i += 64) fdst[i] = ldsf[i];
    for (int i = threadIdx.x; i < 16 * 64; i += 64) hdst[i] = ldsh[i];
}

}  // namespace

extern "C" int hook_wave(int kind, int dtype, const void* in, void* out, int nwaves, void* stream) {
    if (kind < 0 || kind >= kNumKinds || nwaves <= 0) return 1;
    hipStream_t s = (hipStream_t)stream;
    switch (dtype) {
        case 0: wave_kernel<float><<<nwaves, 64, 0, s>>>(kind, (const float*)in, (float*)out); break;
        case 1: wave_kernel_half<__half><<<nwaves, 64, 0, s>>>(kind, (const __half*)in, (float*)out); break;
        case 2: wave_kernel_half<__hip_bfloat16><<<nwaves, 64, 0, s>>>(kind, (const __hip_bfloat16*)in, (float*)out); break;
        case 3: wave_kernel<double><<<nwaves, 64, 0, s>>>(kind, (const double*)in, (double*)out); break;
        case 4: wave_kernel<int32_t><<<nwaves, 64, 0, s>>>(kind, (const int32_t*)in, (int32_t*)out); break;
        case 5: wave_kernel<int64_t><<<nwaves, 64, 0, s>>>(kind, (const int64_t*)in, (int64_t*)out); break;
        default: return 1;
    }
    return (int)hipGetLastError();
}

extern "C" int hook_ballot(const int32_t* in, uint64_t* out, int nwaves, void* stream) {
    ballot_kernel<<<nwaves, 64, 0, (hipStream_t)stream>>>(in, out);
    return (int)hipGetLastError();
}

__global__ void mfma16x4f32_kernel(const float* A, const float* B, float* C) {
    const int lane = threadIdx.x;
    cdna4::mfma::f32x4 c = {0.f, 0.f, 0.f, 0.f};
    c = cdna4::mfma::mma_16x16x4f32(cdna4::mfma::load_A_16x16x4f32(A, lane), cdna4::mfma::load_B_16x16x4f32(B, lane), c);
    cdna4::mfma::store_C_16x16x4f32(C, c, lane);
}

// which: 0 = cdna3::mfma 16x16x16 f16; 1/2 = 16x16x32 f16/bf16; 3/4 = 32x32x16 f16/bf16; 5 = 16x16x4 f32.
extern "C" int hook_mfma(int which, const void* A, const void* B, float* C, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    switch (which) {
        case 0: mfma16_kernel<<<1, 64, 0, s>>>((const __half*)A, (const __half*)B, C); break;
        case 1: mfma16x32_kernel<cdna4::mfma::f16x8, _Float16><<<1, 64, 0, s>>>((const _Float16*)A, (const _Float16*)B, C); break;
        case 2: mfma16x32_kernel<cdna4::mfma::bf16x8, __bf16><<<1, 64, 0, s>>>((const __bf16*)A, (const __bf16*)B, C); break;
        case 3: mfma32x16_kernel<cdna4::mfma::f16x8, _Float16><<<1, 64, 0, s>>>((const _Float16*)A, (const _Float16*)B, C); break;
        case 4: mfma32x16_kernel<cdna4::mfma::bf16x8, __bf16><<<1, 64, 0, s>>>((const __bf16*)A, (const __bf16*)B, C); break;
        case 5: mfma16x4f32_kernel<<<1, 64, 0, s>>>((const float*)A, (const float*)B, C); break;
        default: return 1;
    }
    return (int)hipGetLastError();
}

extern "C" int hook_dme(const void* src, void* dst, const float* fsrc, float* fdst, const void* hsrc, void* hdst,
                        void* stream) {
    dme_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const uint8_t*)src, (uint8_t*)dst, fsrc, fdst, (const __half*)hsrc,
                                                  (__half*)hdst);
    return (int)hipGetLastError();
}

// ---- dme forms the reference's kernels call -------------------------------------------------
// One wave: copy_element / copy_element_stream of lane L's float into tile[L] (the documented
// per-lane form), copy_tile_1d_stream of 256 floats; each tile copied back out.
__global__ void dme_elem_kernel(const float* __restrict__ src, float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) float t0[64];
    __shared__ __attribute__((aligned(16))) float t1[64];
    __shared__ __attribute__((aligned(16))) float t2[256];
    const int L = threadIdx.x;
    dme::copy_element(src + L, &t0[L]);
    dme::copy_element_stream(src + 64 + L, &t1[L]);
    dme::copy_tile_1d_stream<float, 256>(src + 128, t2);
    dme::wait();
    __syncthreads();
    out[L] = t0[L];
    out[64 + L] = t1[L];
    for (int i = L; i < 256; i += 64) out[128 + i] = t2[i];
}

// Two waves: prefetch_tile2d_fp16<32, 64> of one packed tile.
__global__ void dme_tile2d_kernel(const __half* __restrict__ src, __half* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) __half tile[32 * 64];
    dme::prefetch_tile2d_fp16<32, 64>(src, tile, threadIdx.x, blockDim.x);
    dme::wait();
    __syncthreads();
    for (int i = threadIdx.x; i < 32 * 64; i += blockDim.x) out[i] = tile[i];
}

// Two waves: AsyncTile2D<16, 64> ping/pong over n_tiles consecutive tiles; each iteration copies
// the current buffer out while the next tile is in flight.
__global__ void dme_async_tile_kernel(const __half* __restrict__ src, __half* __restrict__ out, int n_tiles) {
    __shared__ __attribute__((aligned(16))) __half buf[2][16 * 64];
    dme::AsyncTile2D<16, 64> t;
    const int tid = threadIdx.x, nt = blockDim.x;
    t.prologue(src, buf, tid, nt);
    for (int j = 0; j < n_tiles; ++j) {
        t.prefetch_next(src, buf, j + 1, n_tiles, tid, nt);
        for (int i = tid; i < 16 * 64; i += nt) out[(size_t)j * 16 * 64 + i] = buf[t.cur()][i];
        t.wait_next(j + 1, n_tiles);
        t.advance();
    }
}

// One wave: online_softmax_step over n_tiles 64-wide tiles of scores s with values v; out = {m,
// l, sum_k softmax(s)_k v_k} after the last tile.
__global__ void online_softmax_kernel(const float* __restrict__ s, const float* __restrict__ v, int n_tiles,
                                      float* __restrict__ out) {
    const int L = threadIdx.x;
    float m = -INFINITY, l = 0.f, acc = 0.f;
    for (int t = 0; t < n_tiles; ++t) {
        float p;
        const float resc = cdna3::ex::online_softmax_step(s[t * 64 + L], m, l, p);
        acc = acc * resc + wave::dpp::reduce_sum_bcast(p * v[t * 64 + L]);
    }
    if (L == 0) {
        out[0] = m;
        out[1] = l;
        out[2] = acc / l;
    }
}

__global__ void mma_tile_kernel(const __half* A, const __half* B, float* C, int ldA, int ldB, int ldC) {
    cdna3::ex::mma_tile_accumulate(A, B, C, threadIdx.x, ldA, ldB, ldC);
}
template <typename T>
__global__ void mma_tile_k32_kernel(const T* A, const T* B, float* C, int ldA, int ldB, int ldC) {
    cdna3::ex::mma_tile_accumulate_k32<T>(A, B, C, threadIdx.x, ldA, ldB, ldC);
}

extern "C" int hook_dme_forms(const float* fsrc, float* fout, const void* hsrc, void* hout, const void* asrc,
                              void* aout, int n_tiles, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    dme_elem_kernel<<<1, 64, 0, s>>>(fsrc, fout);
    dme_tile2d_kernel<<<1, 128, 0, s>>>((const __half*)hsrc, (__half*)hout);
    dme_async_tile_kernel<<<1, 128, 0, s>>>((const __half*)asrc, (__half*)aout, n_tiles);
    return (int)hipGetLastError();
}

extern "C" int hook_online_softmax(const float* s, const float* v, int n_tiles, float* out, void* stream) {
    online_softmax_kernel<<<1, 64, 0, (hipStream_t)stream>>>(s, v, n_tiles, out);
    return (int)hipGetLastError();
}

// which: 0 = mma_tile_accumulate (16x16x16 f16), 1 / 2 = mma_tile_accumulate_k32 f16 / bf16.
extern "C" int hook_mma_tile(int which, const void* A, const void* B, float* C, int ldA, int ldB, int ldC,
                             void* stream) {
    hipStream_t s = (hipStream_t)stream;
    switch (which) {
        case 0: mma_tile_kernel<<<1, 64, 0, s>>>((const __half*)A, (const __half*)B, C, ldA, ldB, ldC); break;
        case 1: mma_tile_k32_kernel<_Float16><<<1, 64, 0, s>>>((const _Float16*)A, (const _Float16*)B, C, ldA, ldB, ldC); break;
        case 2: mma_tile_k32_kernel<__bf16><<<1, 64, 0, s>>>((const __bf16*)A, (const __bf16*)B, C, ldA, ldB, ldC); break;
        default: return 1;
    }
    return (int)hipGetLastError();
}

// The runtime's __global__ kernels of <cdna3/runtime/forward.hpp>, launched as the reference's
// layer loop launches them (session.hpp:168-177, :193-207, :246-249): grid M x 256 threads for the
// norm, one 256-thread block per 256 elements for the rest.
extern "C" int hook_runtime_kernels(int which, const void* a, void* b, const void* c, const void* d, int i0, int i1,
                                    int i2, int i3, int i4, float f, void* stream) {
    using namespace cdna3::runtime;
    hipStream_t s = (hipStream_t)stream;
    auto grid1d = [](long long n) { return dim3((unsigned)((n + 255) / 256)); };
    switch (which) {
        case 0:   // rmsnorm_f32_kernel(X, W, Y, M, H, eps), block i2 threads (the reference: 256)
            hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3(i0), dim3(i2), 0, s, (const float*)a, (const __half*)c,
                               (float*)b, i0, i1, f);
            break;
        case 1:   // rope_kernel(T, cos, sin, seq, heads, D) in place on b
            hipLaunchKernelGGL(rope_kernel, grid1d((long long)i0 * i1 * i2), dim3(256), 0, s, (__half*)b,
                               (const float*)c, (const float*)d, i0, i1, i2);
            break;
        case 2:   // repack_kernel(src, dst, seq, heads, D, dir)
            hipLaunchKernelGGL(repack_kernel, grid1d((long long)i0 * i1 * i2), dim3(256), 0, s, (const __half*)a,
                               (__half*)b, i0, i1, i2, i3);
            break;
        case 3:   // scatter_kv_kernel(src, cache, T, heads, D, pos0, max_seq)
            hipLaunchKernelGGL(scatter_kv_kernel, grid1d((long long)i0 * i1 * i2), dim3(256), 0, s,
                               (const __half*)a, (__half*)b, i0, i1, i2, i3, i4);
            break;
        case 4:   // pack_kv_kernel(cache, packed, heads, N, D, max_seq)
            hipLaunchKernelGGL(pack_kv_kernel, grid1d((long long)i0 * i1 * i2), dim3(256), 0, s, (const __half*)a,
                               (__half*)b, i0, i1, i2, i3);
            break;
        case 5: case 6: case 7: case 8: case 9: {
            // the GEMMs: X = a, W = c, B = d (case 6), Y = b; M = i0, N = i1, K = i2, block i3 x i4
            // (the reference: 16 x 16), grid covering N x M
            const dim3 tb((unsigned)i3, (unsigned)i4), gr((unsigned)((i1 + i3 - 1) / i3), (unsigned)((i0 + i4 - 1) / i4));
            if (which == 5)
                hipLaunchKernelGGL(gemm_f32in_f16out_kernel, gr, tb, 0, s, (const float*)a, (const __half*)c,
                                   (__half*)b, i0, i1, i2);
            else if (which == 6)
                hipLaunchKernelGGL(gemm_f32in_f16out_bias_kernel, gr, tb, 0, s, (const float*)a, (const __half*)c,
                                   (const __half*)d, (__half*)b, i0, i1, i2);
            else if (which == 7)
                hipLaunchKernelGGL(gemm_f32in_f32out_kernel, gr, tb, 0, s, (const float*)a, (const __half*)c,
                                   (float*)b, i0, i1, i2);
            else if (which == 8)
                hipLaunchKernelGGL(gemm_f16in_f32out_kernel, gr, tb, 0, s, (const __half*)a, (const __half*)c,
                                   (float*)b, i0, i1, i2);
            else
                hipLaunchKernelGGL(gemm_xwT_kernel, gr, tb, 0, s, (const __half*)a, (const __half*)c, (__half*)b, i0,
                                   i1, i2);
            break;
        }
        case 10:  // silu_mul_f32_kernel(gate = b, up = a, n = i0), i1 threads per block, grid covering n
            hipLaunchKernelGGL(silu_mul_f32_kernel, dim3((unsigned)((i0 + i1 - 1) / i1)), dim3((unsigned)i1), 0, s,
                               (float*)b, (const float*)a, (size_t)i0);
            break;
        case 11:  // add_f32_kernel(x = b, y = a, n = i0)
            hipLaunchKernelGGL(add_f32_kernel, dim3((unsigned)((i0 + i1 - 1) / i1)), dim3((unsigned)i1), 0, s,
                               (float*)b, (const float*)a, (size_t)i0);
            break;
        case 12:  // embed_gather_f32_kernel(embed = a, ids = c, out = b, T = i0, H = i1), grid T x 256
            hipLaunchKernelGGL(embed_gather_f32_kernel, dim3((unsigned)i0), dim3(256), 0, s, (const __half*)a,
                               (const int*)c, (float*)b, i0, i1);
            break;
        case 13:  // argmax_kernel(logits = a, V = i0, out = b), one block of i1 threads (the reference: 256)
            hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3((unsigned)i1), 0, s, (const __half*)a, i0, (int*)b);
            break;
        default: return 1;
    }
    return (int)hipGetLastError();
}
