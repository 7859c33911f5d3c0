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

}  // namespace runtime
}  // namespace cdna3
