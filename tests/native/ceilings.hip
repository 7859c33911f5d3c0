// Measured ceilings of one MI355X that the design notes compare kernels against (test-only
// program; tests/test_gpu_ceilings.py runs it and prints its line):
//   read_nt / read   a streaming read of a 1 GiB buffer, each workgroup over a contiguous chunk,
//                    with the non-temporal load policy and with the default one;
//   copy_nt          a 1 GiB -> 1 GiB copy, non-temporal loads and stores (read + write bytes);
//   mfma_bf16        back-to-back v_mfma_f32_16x16x32_bf16 on every CU, eight waves per CU,
//                    four independent accumulators per wave, operands rotating over four
//                    preloaded register pairs (no VALU work);
//   mfma_bf16_exp    the same with one v_exp_f32 beside every two MFMAs (the prefill's ratio of
//                    exponentials to matrix instructions);
//   mfma_f16(_exp)   both with v_mfma_f32_16x16x32_f16 on the same bit patterns;
//   lds_dma_cu       the asynchronous global -> LDS copy rate of one CU: eight workgroups of four
//                    waves (one per XCD), each streaming its own 16 MiB through a ring of four
//                    16 KiB LDS stages (three in flight) with global_load_lds_dwordx4, reported per
//                    CU; the 128 MiB are re-read every launch, so they come from the Infinity Cache;
//   lds_dma_nt       the same copy loop on every CU at once, non-temporal (as the decode kernels
//                    copy K/V), over the 1 GiB buffer: the chip's HBM -> LDS rate, best of one or
//                    two workgroups per CU;
// each the median of five timed runs (HIP events), printed as one JSON line. `ceilings mfma S [exp]
// [f16]` instead runs only one MFMA stream for about S seconds, one line per 50 launches.
// The buffer reads are 1 GiB, four times the 256 MB Infinity Cache, so no read is served from it.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>
#include <vector>
#include <cdna3/mfma.hpp>

#define CK(x)                                                                        \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using cdna4::mfma::bf16x8;
using cdna4::mfma::f16x8;
using cdna4::mfma::f32x4;

// Each workgroup reads one contiguous chunk of the buffer (its share, in 256 x U vector steps, the U
// loads of a lane 4 KiB apart), as the decode and reduce kernels stream their key ranges.
template <bool kNT, int U>
__global__ __launch_bounds__(256) void read_stream(const u32x4* __restrict__ p, size_t nvec, uint32_t* sink) {
    const size_t chunk = (nvec + gridDim.x - 1) / gridDim.x;
    const size_t lo = (size_t)blockIdx.x * chunk, hi = lo + chunk < nvec ? lo + chunk : nvec;
    size_t i = lo + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * 256 < hi; i += U * 256) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = kNT ? __builtin_nontemporal_load(p + i + u * 256) : p[i + u * 256];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < hi; i += 256) {
        const u32x4 v = p[i];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;   // keeps the loads; the value never matches here
}

// One workgroup's copy loop of lds_dma_cu: per stage each wave copies 4 KiB (four 1 KiB copies),
// keeps three stages in flight, and waits for the oldest before issuing the next.
template <bool kNT>
__global__ __launch_bounds__(256) void lds_dma(const char* __restrict__ src, size_t per_wg, uint32_t* sink) {
    constexpr int S = 4;
    __shared__ __attribute__((aligned(16))) char lds[S * 16384];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const char* base = src + blockIdx.x * per_wg;
    const int nch = (int)(per_wg / 16384);
    auto issue = [&](int c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const char* g = base + (size_t)c * 16384 + (wave * 4 + j) * 1024 + lane * 16;
            const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(
                lds + (c % S) * 16384 + (wave * 4 + j) * 1024);
            if constexpr (kNT)
                asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(g), "{m0}"(l) : "memory");
            else
                asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(l) : "memory");
        }
    };
    for (int c = 0; c < S - 1 && c < nch; ++c) issue(c);
    for (int c = 0; c < nch; ++c) {
        if (c + S - 1 < nch) {
            issue(c + S - 1);
            asm volatile("s_waitcnt vmcnt(12)" : : : "memory");   // 4 copies x (S - 1) younger stages
        } else {
            asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        }
    }
    if (threadIdx.x == 0 && lds[lane] == 123) sink[0] = 1;   // keeps the copies; never true here
}

template <int U>
__global__ __launch_bounds__(256) void copy_nt(const u32x4* __restrict__ src, u32x4* __restrict__ dst, size_t nvec) {
    const size_t chunk = (nvec + gridDim.x - 1) / gridDim.x;
    const size_t lo = (size_t)blockIdx.x * chunk, hi = lo + chunk < nvec ? lo + chunk : nvec;
    size_t i = lo + threadIdx.x;
    for (; i + (U - 1) * 256 < hi; i += U * 256) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
        for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u], dst + i + u * 256);
    }
    for (; i < hi; i += 256) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

template <bool kExp, class T>
__global__ __launch_bounds__(512) void mfma_stream(const uint32_t* __restrict__ seed, int iters, float* out) {
    const int lane = threadIdx.x & 63;
    T a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        u32x4 wa, wb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            wa[e] = seed[(j * 8 + e) * 64 + lane];
            wb[e] = seed[(j * 8 + 4 + e) * 64 + lane];
        }
        a[j] = __builtin_bit_cast(T, wa);
        b[j] = __builtin_bit_cast(T, wb);
    }
    f32x4 c[4] = {};
    float x[4] = {0.5f, 0.25f, 0.125f, 0.0625f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = cdna4::mfma::mma_16x16x32(a[j], b[(j + r) & 3], c[j]);
                if (kExp && (j & 1)) x[(r * 2 + j / 2) & 3] = __builtin_amdgcn_exp2f(-x[(r * 2 + j / 2) & 3]);
            }
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][1] + c[j][2] + c[j][3] + x[j];
    if (s == 1234.5f) out[0] = s;   // keeps the work; never true here
}

static float median(std::vector<float> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

template <typename F>
static float time_ms(F&& launch, int reps) {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    launch();   // warm-up
    CK(hipDeviceSynchronize());
    std::vector<float> t;
    for (int r = 0; r < reps; ++r) {
        CK(hipEventRecord(e0));
        launch();
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms = 0.f;
        CK(hipEventElapsedTime(&ms, e0, e1));
        t.push_back(ms);
    }
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    return median(t);
}

// `ceilings mfma SECONDS [exp] [f16]`: only one MFMA stream (with the exponentials when `exp` is
// given, fp16 operands when `f16` is), launched back to back for about SECONDS, for sampling board
// power and clocks beside it.
template <class T>
static void launch_mfma(bool with_exp, int cus, const uint32_t* seed, int iters, float* out) {
    if (with_exp) mfma_stream<true, T><<<cus, 512>>>(seed, iters, out);
    else mfma_stream<false, T><<<cus, 512>>>(seed, iters, out);
}

static int mfma_loop(int cus, double seconds, bool with_exp, bool f16) {
    std::vector<uint32_t> h(32 * 64);
    uint32_t s = 12345u;
    for (auto& v : h) {
        s = s * 1664525u + 1013904223u;
        v = (s & 0x807f807fu) | 0x3f003f00u;
    }
    uint32_t* buf = nullptr;
    CK(hipMalloc(&buf, 16384));
    CK(hipMemcpy(buf, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    const int iters = 40000;
    const double flop = (double)cus * 8 * iters * 16 * (2.0 * 16 * 16 * 32);
    float* fout = (float*)(buf + 2048);
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    double total_ms = 0.0;
    long launches = 0;
    while (total_ms < seconds * 1e3) {
        CK(hipEventRecord(e0));
        for (int r = 0; r < 50; ++r) {
            if (f16) launch_mfma<f16x8>(with_exp, cus, buf, iters, fout);
            else launch_mfma<bf16x8>(with_exp, cus, buf, iters, fout);
        }
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms = 0.f;
        CK(hipEventElapsedTime(&ms, e0, e1));
        total_ms += ms;
        launches += 50;
        printf("{\"mfma_loop\": \"%s%s\", \"elapsed_s\": %.1f, \"TFLOPs\": %.1f}\n", f16 ? "f16" : "bf16",
               with_exp ? "+exp" : "", total_ms * 1e-3, 50 * flop / (ms * 1e-3) / 1e12);
        fflush(stdout);
    }
    CK(hipGetLastError());
    CK(hipFree(buf));
    return launches > 0 ? 0 : 1;
}

int main(int argc, char** argv) {
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    const int cus = prop.multiProcessorCount;
    if (argc >= 3 && strcmp(argv[1], "mfma") == 0) {
        bool with_exp = false, f16 = false;
        for (int i = 3; i < argc; ++i) {
            with_exp |= strcmp(argv[i], "exp") == 0;
            f16 |= strcmp(argv[i], "f16") == 0;
        }
        return mfma_loop(cus, atof(argv[2]), with_exp, f16);
    }
    const size_t bytes = (size_t)1 << 30, nvec = bytes / 16;
    u32x4 *a = nullptr, *b = nullptr;
    uint32_t* sink = nullptr;
    CK(hipMalloc(&a, bytes));
    CK(hipMalloc(&b, bytes));
    CK(hipMalloc(&sink, 16384));   // [0, 8 KiB): the MFMA operands (32 x 64 words); 8 KiB on: outputs
    CK(hipMemset(a, 0x5a, bytes));
    CK(hipMemset(b, 0, bytes));
    // Each figure is the best over grids of 4 to 32 workgroups per CU and 4 or 8 loads in flight per
    // lane; the winning shape is printed beside it.
    struct Best { float ms = 1e30f; int grid = 0, u = 0; } r_nt, r_df, c_nt;
    auto keep = [](Best& b, float ms, int grid, int u) { if (ms < b.ms) b = Best{ms, grid, u}; };
    for (int per_cu : {4, 8, 16, 32}) {
        const int grid = cus * per_cu;
        keep(r_nt, time_ms([&] { read_stream<true, 4><<<grid, 256>>>(a, nvec, sink); }, 5), grid, 4);
        keep(r_nt, time_ms([&] { read_stream<true, 8><<<grid, 256>>>(a, nvec, sink); }, 5), grid, 8);
        keep(r_df, time_ms([&] { read_stream<false, 4><<<grid, 256>>>(a, nvec, sink); }, 5), grid, 4);
        keep(r_df, time_ms([&] { read_stream<false, 8><<<grid, 256>>>(a, nvec, sink); }, 5), grid, 8);
        keep(c_nt, time_ms([&] { copy_nt<4><<<grid, 256>>>(a, b, nvec); }, 5), grid, 4);
        keep(c_nt, time_ms([&] { copy_nt<8><<<grid, 256>>>(a, b, nvec); }, 5), grid, 8);
    }
    CK(hipGetLastError());

    std::vector<uint32_t> h(32 * 64);
    uint32_t s = 12345u;
    for (auto& v : h) {   // bf16 pairs with exponents near 1, random mantissas and signs
        s = s * 1664525u + 1013904223u;
        v = (s & 0x807f807fu) | 0x3f003f00u;
    }
    CK(hipMemcpy(sink, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    const int iters = 40000;
    const double flop = (double)cus * 8 * iters * 16 * (2.0 * 16 * 16 * 32);
    float* fout = (float*)(sink + 2048);
    const float m0 = time_ms([&] { launch_mfma<bf16x8>(false, cus, sink, iters, fout); }, 5);
    const float m1 = time_ms([&] { launch_mfma<bf16x8>(true, cus, sink, iters, fout); }, 5);
    const float h0 = time_ms([&] { launch_mfma<f16x8>(false, cus, sink, iters, fout); }, 5);
    const float h1 = time_ms([&] { launch_mfma<f16x8>(true, cus, sink, iters, fout); }, 5);
    const size_t per_wg = (size_t)16 << 20;
    const float dm = time_ms([&] { lds_dma<false><<<8, 256>>>((const char*)a, per_wg, sink + 2048); }, 5);
    // every CU: each workgroup copies its contiguous share of the 1 GiB buffer (whole 16 KiB stages)
    float dn = 1e30f;
    int dn_grid = 0;
    size_t dn_bytes = 0;
    for (int per_cu : {1, 2}) {
        const int grid = cus * per_cu;
        const size_t share = bytes / grid / 16384 * 16384;
        const float ms = time_ms([&] { lds_dma<true><<<grid, 256>>>((const char*)a, share, sink + 2048); }, 5);
        if (share * grid / (ms * 1e-3) > dn_bytes / (dn * 1e-3)) {
            dn = ms;
            dn_grid = grid;
            dn_bytes = share * grid;
        }
    }
    CK(hipGetLastError());
    printf("{\"cus\": %d, \"read_nt_GBs\": %.1f, \"read_GBs\": %.1f, \"copy_nt_GBs\": %.1f, "
           "\"mfma_bf16_TFLOPs\": %.1f, \"mfma_bf16_exp_TFLOPs\": %.1f, \"mfma_f16_TFLOPs\": %.1f, "
           "\"mfma_f16_exp_TFLOPs\": %.1f, \"lds_dma_cu_GBs\": %.1f, \"lds_dma_nt_GBs\": %.1f, "
           "\"shapes\": {\"read_nt\": [%d, %d], \"read\": [%d, %d], \"copy_nt\": [%d, %d], \"lds_dma_nt\": [%d]}}\n",
           cus, bytes / (r_nt.ms * 1e-3) / 1e9, bytes / (r_df.ms * 1e-3) / 1e9, 2.0 * bytes / (c_nt.ms * 1e-3) / 1e9,
           flop / (m0 * 1e-3) / 1e12, flop / (m1 * 1e-3) / 1e12, flop / (h0 * 1e-3) / 1e12,
           flop / (h1 * 1e-3) / 1e12, per_wg / (dm * 1e-3) / 1e9, dn_bytes / (dn * 1e-3) / 1e9, r_nt.grid, r_nt.u,
           r_df.grid, r_df.u, c_nt.grid, c_nt.u, dn_grid);
    CK(hipFree(a));
    CK(hipFree(b));
    CK(hipFree(sink));
    return 0;
}
