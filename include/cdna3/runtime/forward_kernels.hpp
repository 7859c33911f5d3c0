#pragma once
// cdna3/runtime/forward_kernels.hpp — the runtime's __global__ kernels for HIP source (gfx950).
//
// The reference's layer loop launches these from HIP code with hipLaunchKernelGGL
// (cdna3-prims/include/cdna3/runtime/session.hpp:168-177, :193-207, :246-249;
// cdna3-prims/tests/validate_decode_dme.hip includes pack_kv_kernel). Same names, parameter lists
// and launch geometry (any grid/block the reference's callers use), gfx950 designs:
//
//   rmsnorm_f32_kernel   one workgroup per row (grid >= M, blockDim.x a multiple of 64, <= 1024;
//                        the reference launches 256). No LDS and no barrier: every wave of the
//                        workgroup forms the row's sum of squares itself (16-byte loads, the
//                        all-lanes DPP/permlane butterfly), so all waves hold the same scale
//                        without exchanging it; the row's repeated reads hit the cache, HBM sees
//                        it once. The workgroup's threads then write their strided share, as in
//                        the reference (forward.hpp:34-56), y = x * rsqrt(mean(x^2) + eps) * w.
//   rope_kernel          one thread per element as launched by the reference (grid covering
//                        seq * heads * D); the thread of element d < D/2 of a head rotates the
//                        pair (d, d + D/2) and writes both, the threads of d >= D/2 do nothing.
//                        The reference updated the pair from two threads in place, a read/write
//                        race between them (forward.hpp:135-148); here each pair has one owner.
//   repack_kernel, scatter_kv_kernel, pack_kv_kernel
//                        the reference's index maps (forward.hpp:190-239), one element per
//                        thread; scatter_kv skips rows at or past max_seq instead of writing past
//                        the cache slot.
//   gemm_f32in_f16out_kernel, gemm_f32in_f16out_bias_kernel, gemm_f32in_f32out_kernel,
//   gemm_f16in_f32out_kernel, gemm_xwT_kernel
//                        Y[M][N] = X[M][K] W[N][K]^T (+ B[N]), the reference's naive GEMMs
//                        (forward.hpp:70-131) with their launch contract: a 2-D grid whose
//                        workgroup (bx, by) covers rows by*blockDim.y .. and columns
//                        bx*blockDim.x .. (the reference launches 16 x 16 blocks, grid
//                        ((N+15)/16, (M+15)/16); the lm_head call is M = 1). Inside a workgroup
//                        the work is not one output per thread: each wave takes one column and
//                        up to four rows of the tile, its 64 lanes split K with 16-byte loads of
//                        W (8 fp16) and X, and a DPP butterfly sums the lanes, so a W row is
//                        read once per four rows with coalesced loads (the reference's thread
//                        per output walked a W row with one 2-byte load per step). Workgroups
//                        of fewer than 64 threads keep one output per thread.
//   silu_mul_f32_kernel, add_f32_kernel
//                        elementwise over n (forward.hpp:154-170) with the reference's grid (one
//                        thread per element or more); grid-stride over 16-byte vectors when both
//                        arrays are 16-byte aligned, scalar otherwise and for the tail.
//   embed_gather_f32_kernel
//                        one workgroup per token row as the reference launches it (forward.hpp:
//                        174-184), 16-byte fp16 loads widened to two 16-byte fp32 stores.
//   argmax_kernel        one workgroup (the reference launches 256 threads; any power of two up
//                        to 1024) over a fp16 logit row (forward.hpp:244-262), with the
//                        reference's result, ties included: its tree keeps, among equal maxima,
//                        the thread whose index has the smallest bit reversal and, inside a
//                        thread, the first index. Here every element forms one 64-bit key
//                        (order-preserving value bits, the complemented bit-reversed i mod
//                        blockDim, the complemented i / blockDim), so the kernel is a plain max
//                        over keys (DPP butterfly per wave, one LDS word per wave): the same index
//                        whatever order the maxima are combined in. Values <= -1e30 (fp16: -inf)
//                        and NaNs are never chosen, and a row with nothing else gives 0, as in
//                        the reference.
//
// Every kernel has internal linkage, so the header can be included by several translation units
// of one program.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include "../../wave_primitives/wave_reduce_dpp.hpp"

namespace cdna3 {
namespace runtime {

static __global__ void rmsnorm_f32_kernel(const float* __restrict__ X, const __half* __restrict__ W,
                                          float* __restrict__ Y, int M, int H, float eps) {
    const int row = blockIdx.x;
    if (row >= M) return;
    const float* x = X + (size_t)row * H;
    float* y = Y + (size_t)row * H;
    const unsigned lane = threadIdx.x & 63u;
    // 16-byte loads when every row start is 16-byte aligned (the usual case: H % 4 == 0).
    const bool vec = (H & 3) == 0 && (((uintptr_t)X | (uintptr_t)Y) & 15u) == 0 && (((uintptr_t)W) & 7u) == 0;
    float ss = 0.f;
    if (vec) {
        const float4* x4 = (const float4*)x;
        for (int i = (int)lane; i < H / 4; i += 64) {
            const float4 v = x4[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (int i = (int)lane; i < H; i += 64) ss += x[i] * x[i];
    }
    ss = wave::dpp::reduce_sum_bcast(ss);
    const float inv = rsqrtf(ss / (float)H + eps);
    const int nt = (int)blockDim.x;
    if (vec) {
        const float4* x4 = (const float4*)x;
        float4* y4 = (float4*)y;
        const uint2* w4 = (const uint2*)W;
        for (int i = (int)threadIdx.x; i < H / 4; i += nt) {
            const float4 v = x4[i];
            const uint2 wb = w4[i];
            const float w0 = __half2float(__ushort_as_half((unsigned short)(wb.x & 0xffffu)));
            const float w1 = __half2float(__ushort_as_half((unsigned short)(wb.x >> 16)));
            const float w2 = __half2float(__ushort_as_half((unsigned short)(wb.y & 0xffffu)));
            const float w3 = __half2float(__ushort_as_half((unsigned short)(wb.y >> 16)));
            y4[i] = make_float4(v.x * inv * w0, v.y * inv * w1, v.z * inv * w2, v.w * inv * w3);
        }
    } else {
        for (int i = (int)threadIdx.x; i < H; i += nt) y[i] = x[i] * inv * __half2float(W[i]);
    }
}

static __global__ void rope_kernel(__half* __restrict__ T, const float* __restrict__ cos,
                                   const float* __restrict__ sin, int seq, int heads, int D) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)seq * heads * D;
    if (idx >= total) return;
    const int half = D / 2;
    const int d = (int)(idx % D);
    if (d >= half) return;   // the pair (d - D/2, d) belongs to the thread of d - D/2
    const long long s = idx / ((long long)heads * D);
    const long long base = idx - d;
    const float t0 = __half2float(T[base + d]);
    const float t1 = __half2float(T[base + d + half]);
    const float c0 = cos[s * D + d], s0 = sin[s * D + d];
    const float c1 = cos[s * D + d + half], s1 = sin[s * D + d + half];
    T[base + d] = __float2half(t0 * c0 + (-t1) * s0);
    T[base + d + half] = __float2half(t1 * c1 + t0 * s1);
}

static __global__ void repack_kernel(const __half* __restrict__ src, __half* __restrict__ dst, int seq, int heads,
                                     int D, int dir) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)seq * heads * D) return;
    const int d = (int)(idx % D);
    const int h = (int)((idx / D) % heads);
    const long long s = idx / ((long long)heads * D);
    const size_t tok = ((size_t)s * heads + h) * D + d;
    const size_t head = ((size_t)h * seq + s) * D + d;
    if (dir == 0) dst[head] = src[tok];
    else dst[tok] = src[head];
}

static __global__ void scatter_kv_kernel(const __half* __restrict__ src, __half* __restrict__ cache, int T, int heads,
                                         int D, int pos0, int max_seq) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)T * heads * D) return;
    const int d = (int)(idx % D);
    const int h = (int)((idx / D) % heads);
    const long long s = idx / ((long long)heads * D);
    if (pos0 + s >= max_seq || pos0 + s < 0) return;
    cache[((size_t)h * max_seq + (size_t)(pos0 + s)) * D + d] = src[((size_t)s * heads + h) * D + d];
}

static __global__ void pack_kv_kernel(const __half* __restrict__ cache, __half* __restrict__ packed, int heads, int N,
                                      int D, int max_seq) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)heads * N * D) return;
    const int d = (int)(idx % D);
    const long long n = (idx / D) % N;
    const long long h = idx / ((long long)N * D);
    packed[((size_t)h * N + n) * D + d] = cache[((size_t)h * max_seq + n) * D + d];
}

namespace detail {

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__half v) { return __half2float(v); }
__device__ __forceinline__ void store_out(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_out(__half* p, float v) { *p = __float2half(v); }

__device__ __forceinline__ void half8_to_f32(const uint4 b, float (&f)[8]) {
    const unsigned w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __half2float(__ushort_as_half((unsigned short)(w[j] & 0xffffu)));
        f[2 * j + 1] = __half2float(__ushort_as_half((unsigned short)(w[j] >> 16)));
    }
}

// Eight consecutive X values of a row starting at a 16-byte aligned element.
__device__ __forceinline__ void load_x8(const float* p, float (&f)[8]) {
    const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void load_x8(const __half* p, float (&f)[8]) { half8_to_f32(*(const uint4*)p, f); }

// Y = X W^T (+ B) over the tile of this workgroup (see the file header).
template <typename TX, typename TY>
__device__ __forceinline__ void gemm_xwt_tile(const TX* __restrict__ X, const __half* __restrict__ W,
                                              const __half* __restrict__ B, TY* __restrict__ Y, int M, int N,
                                              int K) {
    const int r0 = (int)(blockIdx.y * blockDim.y), c0 = (int)(blockIdx.x * blockDim.x);
    const int rows = min((int)blockDim.y, M - r0), cols = min((int)blockDim.x, N - c0);
    if (rows <= 0 || cols <= 0) return;
    const int nt = (int)(blockDim.x * blockDim.y);
    const int waves = nt / 64;
    if (waves == 0) {   // narrower than a wave: one output per thread, as the reference maps them
        const int row = r0 + (int)threadIdx.y, col = c0 + (int)threadIdx.x;
        if (row >= M || col >= N) return;
        float acc = B ? __half2float(B[col]) : 0.f;
        for (int k = 0; k < K; ++k) acc += to_f32(X[(size_t)row * K + k]) * __half2float(W[(size_t)col * K + k]);
        store_out(Y + (size_t)row * N + col, acc);
        return;
    }
    const int tid = (int)(threadIdx.y * blockDim.x + threadIdx.x);
    const int w = tid >> 6, lane = tid & 63;
    if (w >= waves) return;   // the threads of a partial last wave take no part
    const bool vec = (K & 7) == 0 && ((uintptr_t)X & 15u) == 0 && ((uintptr_t)W & 15u) == 0;
    const int row_groups = (rows + 3) / 4;
    for (int item = w; item < cols * row_groups; item += waves) {
        const int col = c0 + item % cols;
        const int rb = r0 + (item / cols) * 4;
        const int nr = min(4, r0 + rows - rb);
        const __half* wrow = W + (size_t)col * K;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (vec) {
            for (int k = lane * 8; k < K; k += 512) {
                float wf[8];
                half8_to_f32(*(const uint4*)(wrow + k), wf);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (r < nr) {
                        float xf[8];
                        load_x8(X + (size_t)(rb + r) * K + k, xf);
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[r] += xf[j] * wf[j];
                    }
                }
            }
        } else {
            for (int k = lane; k < K; k += 64) {
                const float wk = __half2float(wrow[k]);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < nr) acc[r] += to_f32(X[(size_t)(rb + r) * K + k]) * wk;
            }
        }
        const float bias = B ? __half2float(B[col]) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float s = wave::dpp::reduce_sum_bcast(acc[r]);
            if (lane == 0 && r < nr) store_out(Y + (size_t)(rb + r) * N + col, s + bias);
        }
    }
}

// Order-preserving map of a float onto unsigned integers (-0 and +0 map alike: the reference's
// strict > treats them as equal).
__device__ __forceinline__ unsigned ordered_bits(float v) {
    const unsigned u = v == 0.f ? 0u : __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace detail

static __global__ void gemm_f32in_f16out_kernel(const float* __restrict__ X, const __half* __restrict__ W,
                                                __half* __restrict__ Y, int M, int N, int K) {
    detail::gemm_xwt_tile<float, __half>(X, W, nullptr, Y, M, N, K);
}

static __global__ void gemm_f32in_f16out_bias_kernel(const float* __restrict__ X, const __half* __restrict__ W,
                                                     const __half* __restrict__ B, __half* __restrict__ Y, int M,
                                                     int N, int K) {
    detail::gemm_xwt_tile<float, __half>(X, W, B, Y, M, N, K);
}

static __global__ void gemm_f32in_f32out_kernel(const float* __restrict__ X, const __half* __restrict__ W,
                                                float* __restrict__ Y, int M, int N, int K) {
    detail::gemm_xwt_tile<float, float>(X, W, nullptr, Y, M, N, K);
}

static __global__ void gemm_f16in_f32out_kernel(const __half* __restrict__ X, const __half* __restrict__ W,
                                                float* __restrict__ Y, int M, int N, int K) {
    detail::gemm_xwt_tile<__half, float>(X, W, nullptr, Y, M, N, K);
}

static __global__ void gemm_xwT_kernel(const __half* __restrict__ X, const __half* __restrict__ W,
                                       __half* __restrict__ Y, int M, int N, int K) {
    detail::gemm_xwt_tile<__half, __half>(X, W, nullptr, Y, M, N, K);
}

static __global__ void silu_mul_f32_kernel(float* __restrict__ gate, const float* __restrict__ up, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t i0 = 0;
    if ((((uintptr_t)gate | (uintptr_t)up) & 15u) == 0) {
        float4* g4 = (float4*)gate;
        const float4* u4 = (const float4*)up;
        const size_t nv = n / 4;
        for (size_t i = tid; i < nv; i += step) {
            const float4 g = g4[i], u = u4[i];
            g4[i] = make_float4((g.x / (1.f + expf(-g.x))) * u.x, (g.y / (1.f + expf(-g.y))) * u.y,
                                (g.z / (1.f + expf(-g.z))) * u.z, (g.w / (1.f + expf(-g.w))) * u.w);
        }
        i0 = nv * 4;
    }
    for (size_t i = i0 + tid; i < n; i += step) {
        const float g = gate[i];
        gate[i] = (g / (1.f + expf(-g))) * up[i];
    }
}

static __global__ void add_f32_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t i0 = 0;
    if ((((uintptr_t)x | (uintptr_t)y) & 15u) == 0) {
        float4* x4 = (float4*)x;
        const float4* y4 = (const float4*)y;
        const size_t nv = n / 4;
        for (size_t i = tid; i < nv; i += step) {
            const float4 a = x4[i], b = y4[i];
            x4[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        }
        i0 = nv * 4;
    }
    for (size_t i = i0 + tid; i < n; i += step) x[i] += y[i];
}

static __global__ void embed_gather_f32_kernel(const __half* __restrict__ embed, const int* __restrict__ ids,
                                               float* __restrict__ out, int T, int H) {
    const int t = (int)blockIdx.x;
    if (t >= T) return;
    const __half* src = embed + (size_t)ids[t] * H;
    float* dst = out + (size_t)t * H;
    const int nt = (int)blockDim.x;
    int i0 = 0;
    if ((H & 7) == 0 && ((uintptr_t)embed & 15u) == 0 && ((uintptr_t)out & 15u) == 0) {
        for (int i = (int)threadIdx.x; i < H / 8; i += nt) {
            float f[8];
            detail::half8_to_f32(((const uint4*)src)[i], f);
            ((float4*)dst)[2 * i] = make_float4(f[0], f[1], f[2], f[3]);
            ((float4*)dst)[2 * i + 1] = make_float4(f[4], f[5], f[6], f[7]);
        }
        i0 = H;
    }
    for (int i = i0 + (int)threadIdx.x; i < H; i += nt) dst[i] = __half2float(src[i]);
}

static __global__ void argmax_kernel(const __half* __restrict__ logits, int V, int* __restrict__ out) {
    __shared__ unsigned long long best[16];
    const unsigned nt = blockDim.x, t = threadIdx.x;
    const unsigned lg = 31u - (unsigned)__builtin_clz(nt);          // log2 of the block size
    const unsigned idx_bits = 32u - lg;                                // bits left for i / nt
    const unsigned long long idx_mask = (1ull << idx_bits) - 1ull;
    // Thread t sees i = t, t + nt, ...; among tied threads the reference keeps the one whose
    // index has the smallest bit reversal (over lg bits), inside a thread the smallest i / nt.
    auto rank_of = [lg](unsigned x) { return lg ? (__builtin_bitreverse32(x) >> (32u - lg)) : 0u; };
    auto key_of = [&](int i) -> unsigned long long {
        const float v = __half2float(logits[i]);
        if (!(v > -1e30f)) return 0ull;                                // never chosen; NaN too
        const unsigned long long r = ~(unsigned long long)rank_of((unsigned)i & (nt - 1u)) & (nt - 1u);
        return ((unsigned long long)detail::ordered_bits(v) << 32) | (r << idx_bits) |
               (~(unsigned long long)((unsigned)i >> lg) & idx_mask);
    };
    unsigned long long key = 0;    // 0: nothing chosen (every real key has its top bit set)
    if ((nt & 63u) == 0) {         // whole waves
        for (int i = (int)t; i < V; i += (int)nt) {
            const unsigned long long k = key_of(i);
            key = k > key ? k : key;
        }
        key = wave::dpp::reduce_max_bcast(key);
        if ((t & 63u) == 0) best[t >> 6] = key;
        __syncthreads();
        if (t != 0) return;
        for (unsigned w = 1; w < nt / 64u; ++w) key = best[w] > key ? best[w] : key;
    } else {                       // a block with a partial wave: thread 0 scans the row
        if (t != 0) return;
        for (int i = 0; i < V; ++i) {
            const unsigned long long k = key_of(i);
            key = k > key ? k : key;
        }
    }
    if (key == 0) {
        *out = 0;
        return;
    }
    const unsigned winner_t = rank_of((unsigned)(~(key >> idx_bits)) & (nt - 1u));
    const unsigned q = (unsigned)(~key & idx_mask);
    *out = (int)(q * nt + winner_t);
}

}  // namespace runtime
}  // namespace cdna3
