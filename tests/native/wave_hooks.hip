// Test hooks (tests only, not part of libcdna4_attn.so): run the header-only device templates
// of include/ (wave::dpp, wave::, cdna3::mfma, cdna4::mfma, dme::, cdna3::ex) on whole waves so
// that pytest can check them lane by lane against closed forms and the CPU oracle.
#include <hip/hip_runtime.h>
#include <cdna3/cdna3.hpp>
#include <cdna3/examples/fused_softmax.hpp>
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
