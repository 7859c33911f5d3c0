#pragma once
// cdna3/runtime/forward.hpp — the runtime's norm, RoPE and KV-layout entry points (gfx950).
//
// The reference's layer loop launches __global__ kernels from this header directly
// (cdna3-prims/include/cdna3/runtime/forward.hpp:34-56 rmsnorm_f32_kernel, :135-148 rope_kernel,
// :190-239 repack / scatter_kv / pack_kv kernels; launched by session.hpp:168-250). Two forms:
//   * host functions over libcdna4_attn.so (any host compiler), e.g.
//       cdna3::runtime::rmsnorm_f32(X, W, Y, M, H, eps, s)
//       cdna3::runtime::rope_f16(T, cos, sin, seq, heads, D, s)
//     plus the device-side fill_rope (rope_table_f32) and the fused RoPE + K/V append;
//   * in HIP source (hipcc), the kernels themselves under the reference's names and signatures,
//     so code that does
//       hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3(M), dim3(256), 0, s, X, W, Y, M, H, eps)
//       hipLaunchKernelGGL(rope_kernel, dim3((seq*heads*D + 255)/256), dim3(256), 0, s, T, cos, sin,
//                          seq, heads, D)
//     compiles and runs unchanged on gfx950 (see forward_kernels.hpp for their design).
#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include "../../cdna4_attn.h"
#if defined(__HIP__)
#include "forward_kernels.hpp"
#endif

namespace cdna3 {
namespace runtime {

inline hipError_t rmsnorm_f32(const float* X, const __half* W, float* Y, int M, int H, float eps,
                              hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_rmsnorm_f32(X, W, Y, M, H, eps, (cdna4_stream_t)stream);
}
inline hipError_t layernorm_f32(const float* X, const float* gamma, const float* beta, float* Y, int M, int H,
                                float eps = 1e-5f, hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_layernorm_f32(X, gamma, beta, Y, M, H, eps, (cdna4_stream_t)stream);
}
// Row softmax of M rows of H fp32 values (bench_softmax.hip:59-105's softmax_kernel); X may equal Y.
inline hipError_t softmax_rows_f32(const float* X, float* Y, int M, int H, hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_softmax_rows_f32(X, Y, M, H, (cdna4_stream_t)stream);
}
inline hipError_t rope_f16(__half* T, const float* cos, const float* sin, int seq, int heads, int D,
                           hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_rope_f16(T, cos, sin, seq, heads, D, (cdna4_stream_t)stream);
}
// Device-side fill_rope: cos/sin [T][D] for absolute positions pos0 .. pos0 + T - 1.
inline hipError_t rope_table_f32(float* cos, float* sin, int pos0, int T, int D, float theta,
                                 hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_rope_table_f32(cos, sin, pos0, T, D, theta, (cdna4_stream_t)stream);
}

// KV cache and layouts (forward.hpp:190-220 of the reference; Session::append_kv):
//   hipLaunchKernelGGL(scatter_kv_kernel, grid, 256, 0, s, src, cache, T, heads, D, pos0, max_seq)
//     -> cdna3::runtime::scatter_kv_f16(src, cache, T, heads, D, pos0, max_seq, s)
//   hipLaunchKernelGGL(repack_kernel, grid, 256, 0, s, src, dst, seq, heads, D, dir)
//     -> cdna3::runtime::repack_f16(src, dst, seq, heads, D, dir, s)
// and the layer loop's rope_kernel x 2 + Q repack + append_kv in one launch:
//     -> cdna3::runtime::rope_append_kv_f16(q, k, v, q_head, K_layer, V_layer, cos, sin, T, nQH,
//                                            nKVH, D, pos0, max_seq, s)
inline hipError_t scatter_kv_f16(const __half* src, __half* cache, int T, int heads, int D, int pos0, int max_seq,
                                 hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_scatter_kv_f16(src, cache, T, heads, D, pos0, max_seq, (cdna4_stream_t)stream);
}
inline hipError_t repack_f16(const __half* src, __half* dst, int seq, int heads, int D, int dir,
                             hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_repack_f16(src, dst, seq, heads, D, dir, (cdna4_stream_t)stream);
}
inline hipError_t rope_append_kv_f16(const __half* q, const __half* k, const __half* v, __half* q_head,
                                     __half* K_cache, __half* V_cache, const float* cos, const float* sin, int T,
                                     int nQH, int nKVH, int D, int pos0, int max_seq, hipStream_t stream = nullptr) {
    return (hipError_t)cdna3_rope_append_kv_f16(q, k, v, q_head, K_cache, V_cache, cos, sin, T, nQH, nKVH, D, pos0,
                                                max_seq, (cdna4_stream_t)stream);
}

}  // namespace runtime
}  // namespace cdna3
