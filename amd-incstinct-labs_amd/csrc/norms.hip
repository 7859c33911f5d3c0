// Runtime norm and RoPE entry points for gfx950: RMSNorm, two-pass LayerNorm and row softmax with
// one wave per row (DPP/permlane butterfly reductions, zero LDS), rotate-half RoPE with one
// thread per (d, d + D/2) pair, and the RoPE cos/sin table built on the device.
//
// Reference behaviour restated:
//   rmsnorm_f32_kernel  cdna3-prims/include/cdna3/runtime/forward.hpp:34-56
//   layernorm_kernel    research/wave-primitives/benchmarks/bench_layernorm.hip:51-114
//   softmax_kernel<DPP> research/wave-primitives/benchmarks/bench_softmax.hip:59-105
//   rope_kernel         cdna3-prims/include/cdna3/runtime/forward.hpp:135-148
//   Session::fill_rope  cdna3-prims/include/cdna3/runtime/session.hpp:120-135
#include "common.hpp"
#include "wave_primitives/detail/xlane.hpp"

namespace cdna4 {
namespace {

using wave::xlane::allreduce;
using wave::xlane::Max;
using wave::xlane::row_allreduce;
using wave::xlane::Sum;

constexpr int kNormWaves = 4;   // rows per 256-thread block, one wave per row

// X rows and Y rows move as 16-byte vectors; kNT gives them the non-temporal (streaming) cache
// policy, which the launchers choose for tensors of kStreamBytes or more: X and Y of 65536 x 512
// f32, each 134 MB and rotated through 1 GiB, took 44.6 us instead of 49.4 (LayerNorm) with it.
// Smaller tensors keep the default policy, so that a consumer right after the norm can still find
// Y in the Infinity Cache (and the 65536 x 64 shape gained nothing from loads alone).
constexpr size_t kStreamBytes = (size_t)64 << 20;
typedef float f32v4 __attribute__((ext_vector_type(4)));
template <bool kNT>
__device__ __forceinline__ float4 ld4(const float* p) {
    if constexpr (kNT) {
        const f32v4 v = __builtin_nontemporal_load((const f32v4*)p);
        return make_float4(v[0], v[1], v[2], v[3]);
    } else {
        return *(const float4*)p;
    }
}
template <bool kNT>
__device__ __forceinline__ void st4(float* p, float4 o) {
    if constexpr (kNT) __builtin_nontemporal_store(f32v4{o.x, o.y, o.z, o.w}, (f32v4*)p);
    else *(float4*)p = o;
}

// Row cached in registers: NV float4 per lane covers H <= 256 * NV (H % 4 == 0).
template <int NV, bool kNT>
__device__ __forceinline__ void load_row(const float* __restrict__ x, int H, unsigned lane, float4 (&v)[NV]) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        v[k] = (c < H) ? ld4<kNT>(x + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int NV, bool kNT>
__global__ __launch_bounds__(256) void rmsnorm_vec(const float* __restrict__ X, const uint16_t* __restrict__ W,
                                                   float* __restrict__ Y, int M, int H, float eps) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float4 v[NV];
    load_row<NV, kNT>(x, H, lane, v);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
    ss = allreduce(ss, Sum{});
    const float inv = rsqrtf(ss / (float)H + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        if (c < H) {
            const uint2 wb = *(const uint2*)(W + c);
            float4 o;
            o.x = v[k].x * inv * f16_bits_to_f32(wb.x & 0xffffu);
            o.y = v[k].y * inv * f16_bits_to_f32(wb.x >> 16);
            o.z = v[k].z * inv * f16_bits_to_f32(wb.y & 0xffffu);
            o.w = v[k].w * inv * f16_bits_to_f32(wb.y >> 16);
            st4<kNT>(y + c, o);
        }
    }
}

// H <= 64 (H % 4 == 0): one 16-lane DPP row per norm row, four rows per wave, one float4 per lane,
// so short rows keep all 64 lanes busy; each 16-lane row takes kRowsPerLane norm rows kRows16
// apart (a block's r-th loads are one contiguous run), all of its loads issued before any
// arithmetic. Lanes of rows past M run on zeros (the row reductions need every lane of the row)
// and store nothing.
constexpr int kRows16 = 16;      // rows per 256-thread block and load
// Norm rows per 16-lane row: at 65536 x 64 (f32, inputs from HBM) 1 / 2 / 4 / 8 took LayerNorm
// 7.83 / 7.35 / 7.95 / 8.67 us and RMSNorm 7.66 / 7.25 / 7.24 / 7.77 us.
constexpr int kRowsPerLane = 2;
template <bool kNT>
__global__ __launch_bounds__(256) void rmsnorm_row16(const float* __restrict__ X, const uint16_t* __restrict__ W,
                                                     float* __restrict__ Y, int M, int H, float eps) {
    const int c = (int)(threadIdx.x & 15u) * 4;
    const int row0 = blockIdx.x * (kRows16 * kRowsPerLane) + (int)(threadIdx.x >> 4);
    float4 v[kRowsPerLane];
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        v[r] = row < M && c < H ? ld4<kNT>(X + (size_t)row * H + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const uint2 wb = c < H ? *(const uint2*)(W + c) : make_uint2(0u, 0u);
    const float w0 = f16_bits_to_f32(wb.x & 0xffffu), w1 = f16_bits_to_f32(wb.x >> 16);
    const float w2 = f16_bits_to_f32(wb.y & 0xffffu), w3 = f16_bits_to_f32(wb.y >> 16);
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        const float ss =
            row_allreduce((v[r].x * v[r].x + v[r].y * v[r].y) + (v[r].z * v[r].z + v[r].w * v[r].w), Sum{});
        const float inv = rsqrtf(ss / (float)H + eps);
        if (row < M && c < H) {
            float4 o;
            o.x = v[r].x * inv * w0;
            o.y = v[r].y * inv * w1;
            o.z = v[r].z * inv * w2;
            o.w = v[r].w * inv * w3;
            st4<kNT>(Y + (size_t)row * H + c, o);
        }
    }
}

// Any H and alignment: two passes over the row (the second pass hits the cache).
__global__ __launch_bounds__(256) void rmsnorm_any(const float* __restrict__ X, const uint16_t* __restrict__ W,
                                                   float* __restrict__ Y, int M, int H, float eps) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float ss = 0.f;
    for (int c = lane; c < H; c += 64) ss += x[c] * x[c];
    ss = allreduce(ss, Sum{});
    const float inv = rsqrtf(ss / (float)H + eps);
    for (int c = lane; c < H; c += 64) y[c] = x[c] * inv * f16_bits_to_f32(W[c]);
}

template <int NV, bool kNT>
__global__ __launch_bounds__(256) void layernorm_vec(const float* __restrict__ X, const float* __restrict__ G,
                                                     const float* __restrict__ B, float* __restrict__ Y, int M,
                                                     int H, float eps) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float4 v[NV];
    load_row<NV, kNT>(x, H, lane, v);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    const float mean = allreduce(s, Sum{}) / (float)H;
    // Second pass over the register-cached deviations (padding lanes contribute 0).
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        if (c < H) {
            const float a = v[k].x - mean, b = v[k].y - mean, d = v[k].z - mean, e = v[k].w - mean;
            q += (a * a + b * b) + (d * d + e * e);
        }
    }
    const float inv = rsqrtf(allreduce(q, Sum{}) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        if (c < H) {
            const float4 g = *(const float4*)(G + c), bb = *(const float4*)(B + c);
            float4 o;
            o.x = (v[k].x - mean) * inv * g.x + bb.x;
            o.y = (v[k].y - mean) * inv * g.y + bb.y;
            o.z = (v[k].z - mean) * inv * g.z + bb.z;
            o.w = (v[k].w - mean) * inv * g.w + bb.w;
            st4<kNT>(y + c, o);
        }
    }
}

template <bool kNT>
__global__ __launch_bounds__(256) void layernorm_row16(const float* __restrict__ X, const float* __restrict__ G,
                                                       const float* __restrict__ B, float* __restrict__ Y, int M,
                                                       int H, float eps) {
    const int c = (int)(threadIdx.x & 15u) * 4;
    const int row0 = blockIdx.x * (kRows16 * kRowsPerLane) + (int)(threadIdx.x >> 4);
    float4 v[kRowsPerLane];
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        v[r] = row < M && c < H ? ld4<kNT>(X + (size_t)row * H + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float4 g = c < H ? *(const float4*)(G + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 bb = c < H ? *(const float4*)(B + c) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        const float mean = row_allreduce((v[r].x + v[r].y) + (v[r].z + v[r].w), Sum{}) / (float)H;
        // Second pass over the register-cached deviations (padding lanes contribute 0).
        float q = 0.f;
        if (c < H) {
            const float a = v[r].x - mean, b = v[r].y - mean, d = v[r].z - mean, e = v[r].w - mean;
            q = (a * a + b * b) + (d * d + e * e);
        }
        const float inv = rsqrtf(row_allreduce(q, Sum{}) / (float)H + eps);
        if (row < M && c < H) {
            float4 o;
            o.x = (v[r].x - mean) * inv * g.x + bb.x;
            o.y = (v[r].y - mean) * inv * g.y + bb.y;
            o.z = (v[r].z - mean) * inv * g.z + bb.z;
            o.w = (v[r].w - mean) * inv * g.w + bb.w;
            st4<kNT>(Y + (size_t)row * H + c, o);
        }
    }
}

__global__ __launch_bounds__(256) void layernorm_any(const float* __restrict__ X, const float* __restrict__ G,
                                                     const float* __restrict__ B, float* __restrict__ Y, int M,
                                                     int H, float eps) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float s = 0.f;
    for (int c = lane; c < H; c += 64) s += x[c];
    const float mean = allreduce(s, Sum{}) / (float)H;
    float q = 0.f;
    for (int c = lane; c < H; c += 64) { const float d = x[c] - mean; q += d * d; }
    const float inv = rsqrtf(allreduce(q, Sum{}) / (float)H + eps);
    for (int c = lane; c < H; c += 64) y[c] = (x[c] - mean) * inv * G[c] + B[c];
}

// ---- row softmax: y = exp(x - max(x)) / sum(exp(x - max(x))) per row ------------------------
// The reference's order of work: the row maximum (DPP max), exp(x - m) (__expf), their sum (DPP
// sum), then each value times 1 / sum. Columns past H take -inf into the maximum and 0 into the
// sum. Same row layouts as the norms: one wave per row with the row in registers (H <= 256 NV),
// 16 lanes per row for H <= 64, two passes for anything else.
template <int NV, bool kNT>
__global__ __launch_bounds__(256) void softmax_vec(const float* __restrict__ X, float* __restrict__ Y, int M, int H) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        v[k] = (c < H) ? ld4<kNT>(x + c) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) m = fmaxf(fmaxf(m, fmaxf(v[k].x, v[k].y)), fmaxf(v[k].z, v[k].w));
    m = allreduce(m, Max{});
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        v[k] = make_float4(__expf(v[k].x - m), __expf(v[k].y - m), __expf(v[k].z - m), __expf(v[k].w - m));
        sum += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float inv = 1.f / allreduce(sum, Sum{});
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = (k * 64 + (int)lane) * 4;
        if (c < H) st4<kNT>(y + c, make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv));
    }
}

template <bool kNT>
__global__ __launch_bounds__(256) void softmax_row16(const float* __restrict__ X, float* __restrict__ Y, int M, int H) {
    const int c = (int)(threadIdx.x & 15u) * 4;
    const int row0 = blockIdx.x * (kRows16 * kRowsPerLane) + (int)(threadIdx.x >> 4);
    float4 v[kRowsPerLane];
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        v[r] = row < M && c < H ? ld4<kNT>(X + (size_t)row * H + c)
                                : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) {
        const int row = row0 + r * kRows16;
        float m = row_allreduce(fmaxf(fmaxf(v[r].x, v[r].y), fmaxf(v[r].z, v[r].w)), Max{});
        if (m == -INFINITY) m = 0.f;   // rows past M: all -inf, kept finite (nothing is stored)
        const float4 e = make_float4(__expf(v[r].x - m), __expf(v[r].y - m), __expf(v[r].z - m), __expf(v[r].w - m));
        const float inv = 1.f / row_allreduce((e.x + e.y) + (e.z + e.w), Sum{});
        if (row < M && c < H) st4<kNT>(Y + (size_t)row * H + c, make_float4(e.x * inv, e.y * inv, e.z * inv, e.w * inv));
    }
}

// Reads each value three times and may run in place (X == Y), so X and Y are not restrict.
__global__ __launch_bounds__(256) void softmax_any(const float* X, float* Y, int M, int H) {
    const unsigned lane = threadIdx.x & 63u;
    const int row = blockIdx.x * kNormWaves + (int)(threadIdx.x >> 6);
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    float m = -INFINITY;
    for (int c = lane; c < H; c += 64) m = fmaxf(m, x[c]);
    m = allreduce(m, Max{});
    float s = 0.f;
    for (int c = lane; c < H; c += 64) s += __expf(x[c] - m);
    const float inv = 1.f / allreduce(s, Sum{});
    for (int c = lane; c < H; c += 64) y[c] = __expf(x[c] - m) * inv;
}

// One thread per (row, head, d) with d < D/2: reads t[d] and t[d + D/2] once, writes both.
__global__ __launch_bounds__(256) void rope_pairs(uint16_t* __restrict__ T, const float* __restrict__ cosv,
                                                  const float* __restrict__ sinv, int seq, int heads, int D) {
    const int half = D >> 1;
    const size_t total = (size_t)seq * heads * half;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int d = (int)(idx % half);
    const size_t sh = idx / half;               // s * heads + h
    const int s = (int)(sh / heads);
    uint16_t* t = T + sh * D;
    const float* c = cosv + (size_t)s * D;
    const float* sn = sinv + (size_t)s * D;
    const float a = f16_bits_to_f32(t[d]);
    const float b = f16_bits_to_f32(t[d + half]);
    const float lo = a * c[d] + (-b) * sn[d];
    const float hi = b * c[d + half] + a * sn[d + half];
    t[d] = (uint16_t)f32_to_f16_bits(lo);
    t[d + half] = (uint16_t)f32_to_f16_bits(hi);
}

__global__ __launch_bounds__(256) void rope_table(float* __restrict__ cosv, float* __restrict__ sinv, int pos0,
                                                  int T, int D, float theta) {
    const int half = D >> 1;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)T * half) return;
    const int d = (int)(idx % half);
    const int s = (int)(idx / half);
    const float freq = 1.f / powf(theta, (2.f * (float)d) / (float)D);
    const float ang = (float)(pos0 + s) * freq;
    const float cv = cosf(ang), sv = sinf(ang);
    cosv[(size_t)s * D + d] = cv;
    cosv[(size_t)s * D + d + half] = cv;
    sinv[(size_t)s * D + d] = sv;
    sinv[(size_t)s * D + d + half] = sv;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <class Launch>
int dispatch_nv(int H, Launch&& launch) {
    if (H <= 256) return launch(std::integral_constant<int, 1>{});
    if (H <= 512) return launch(std::integral_constant<int, 2>{});
    if (H <= 1024) return launch(std::integral_constant<int, 4>{});
    if (H <= 2048) return launch(std::integral_constant<int, 8>{});
    return launch(std::integral_constant<int, 16>{});
}

}  // namespace
}  // namespace cdna4

using namespace cdna4;

extern "C" int cdna3_rmsnorm_f32(const float* X, const void* W, float* Y, int M, int H, float eps,
                                 cdna4_stream_t stream) {
    if (M < 0 || H <= 0 || (M > 0 && (!X || !W || !Y))) return CDNA4_ERR_INVALID_VALUE;
    if (M == 0) return 0;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = ceil_div((size_t)M, kNormWaves);
    const uint16_t* w = (const uint16_t*)W;
    const bool vec = (H % 4 == 0) && H <= 4096 && aligned16(X) && aligned16(Y) && (((uintptr_t)W & 7u) == 0);
    if (!vec) {
        rmsnorm_any<<<grid, 256, 0, s>>>(X, w, Y, M, H, eps);
        return launch_status();
    }
    const bool nt = (size_t)M * (size_t)H * sizeof(float) >= kStreamBytes;
    if (H <= 64) {
        if (nt) rmsnorm_row16<true><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, w, Y, M, H, eps);
        else rmsnorm_row16<false><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, w, Y, M, H, eps);
        return launch_status();
    }
    return dispatch_nv(H, [&](auto nv) {
        if (nt) rmsnorm_vec<decltype(nv)::value, true><<<grid, 256, 0, s>>>(X, w, Y, M, H, eps);
        else rmsnorm_vec<decltype(nv)::value, false><<<grid, 256, 0, s>>>(X, w, Y, M, H, eps);
        return launch_status();
    });
}

extern "C" int cdna3_layernorm_f32(const float* X, const float* gamma, const float* beta, float* Y, int M, int H,
                                   float eps, cdna4_stream_t stream) {
    if (M < 0 || H <= 0 || (M > 0 && (!X || !gamma || !beta || !Y))) return CDNA4_ERR_INVALID_VALUE;
    if (M == 0) return 0;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = ceil_div((size_t)M, kNormWaves);
    const bool vec = (H % 4 == 0) && H <= 4096 && aligned16(X) && aligned16(Y) && aligned16(gamma) && aligned16(beta);
    if (!vec) {
        layernorm_any<<<grid, 256, 0, s>>>(X, gamma, beta, Y, M, H, eps);
        return launch_status();
    }
    const bool nt = (size_t)M * (size_t)H * sizeof(float) >= kStreamBytes;
    if (H <= 64) {
        if (nt) layernorm_row16<true><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, gamma, beta, Y, M, H, eps);
        else layernorm_row16<false><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, gamma, beta, Y, M, H, eps);
        return launch_status();
    }
    return dispatch_nv(H, [&](auto nv) {
        if (nt) layernorm_vec<decltype(nv)::value, true><<<grid, 256, 0, s>>>(X, gamma, beta, Y, M, H, eps);
        else layernorm_vec<decltype(nv)::value, false><<<grid, 256, 0, s>>>(X, gamma, beta, Y, M, H, eps);
        return launch_status();
    });
}

extern "C" int cdna3_softmax_rows_f32(const float* X, float* Y, int M, int H, cdna4_stream_t stream) {
    if (M < 0 || H <= 0 || (M > 0 && (!X || !Y))) return CDNA4_ERR_INVALID_VALUE;
    if (M == 0) return 0;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = ceil_div((size_t)M, kNormWaves);
    const bool vec = (H % 4 == 0) && H <= 4096 && aligned16(X) && aligned16(Y);
    if (!vec) {
        softmax_any<<<grid, 256, 0, s>>>(X, Y, M, H);
        return launch_status();
    }
    const bool nt = (size_t)M * (size_t)H * sizeof(float) >= kStreamBytes;
    if (H <= 64) {
        if (nt) softmax_row16<true><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, Y, M, H);
        else softmax_row16<false><<<ceil_div((size_t)M, kRows16 * kRowsPerLane), 256, 0, s>>>(X, Y, M, H);
        return launch_status();
    }
    return dispatch_nv(H, [&](auto nv) {
        if (nt) softmax_vec<decltype(nv)::value, true><<<grid, 256, 0, s>>>(X, Y, M, H);
        else softmax_vec<decltype(nv)::value, false><<<grid, 256, 0, s>>>(X, Y, M, H);
        return launch_status();
    });
}

extern "C" int cdna3_rope_f16(void* T, const float* cos_tab, const float* sin_tab, int seq, int heads, int D,
                              cdna4_stream_t stream) {
    if (seq < 0 || heads <= 0 || D <= 0 || (D & 1)) return CDNA4_ERR_INVALID_VALUE;
    if (seq == 0) return 0;
    if (!T || !cos_tab || !sin_tab) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    const size_t total = (size_t)seq * heads * (D / 2);
    rope_pairs<<<ceil_div(total, 256), 256, 0, (hipStream_t)stream>>>((uint16_t*)T, cos_tab, sin_tab, seq, heads, D);
    return launch_status();
}

extern "C" int cdna3_rope_table_f32(float* cos_tab, float* sin_tab, int pos0, int T, int D, float theta,
                                    cdna4_stream_t stream) {
    if (T < 0 || D <= 0 || (D & 1) || pos0 < 0 || !(theta > 0.f)) return CDNA4_ERR_INVALID_VALUE;
    if (T == 0) return 0;
    if (!cos_tab || !sin_tab) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    const size_t total = (size_t)T * (D / 2);
    rope_table<<<ceil_div(total, 256), 256, 0, (hipStream_t)stream>>>(cos_tab, sin_tab, pos0, T, D, theta);
    return launch_status();
}
