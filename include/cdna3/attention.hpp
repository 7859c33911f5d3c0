#pragma once
// cdna3/attention.hpp — cdna3::attn host launchers (gfx950), drop-in for the reference's
// cdna3-prims/include/cdna3/attention.hpp:63-173.
//
// Same structs, names, argument order, default stream and hipError_t returns as the
// reference. The kernels live in libcdna4_attn.so behind its C ABI (cdna4_attn.h); these
// inline wrappers only translate the call. Link with -lcdna4_attn. Host-only: this header
// compiles with g++ (-D__HIP_PLATFORM_AMD__ -I/opt/rocm/include) as well as with hipcc.
//
// Behaviour differences from the reference, all documented in cdna4_attn.h:
//   * any seqQ / seqK >= 1 is computed in full (the reference silently truncated shapes that
//     were not multiples of its tiles); causal requires seqQ == seqK;
//   * decode and decode_dme without a workspace run one launch that needs no memory beyond
//     q, K, V and o, like the reference's (no allocation, nothing shared between calls): one
//     workgroup per (batch, kv head, group of 16 query heads), so a few long sequences run on
//     that many CUs. Measured on one MI355X at the reference's decode benchmark shape (batch 1,
//     32 q / 8 kv heads, D 128, fp16): 74 us at N 8192, 41 us at N 4096. The overloads taking
//     (workspace, bytes) split long caches over a split-K grid instead: 11-14 / 9-15 us at the
//     same shapes (decode_workspace_size gives the bytes, 1.06 MB there). Use them whenever
//     batch x nKVHeads is well below the device's CU count.
// New overloads: bf16 tensors, a batch dimension (DecodeCfg::batch), fp32 prefill, split-K
// workspaces.
#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include "../cdna4_attn.h"

namespace cdna3 {
namespace attn {

struct PrefillCfg {
    int D;          // head dimension (64 or 128)
    int seqQ;       // query sequence length
    int seqK;       // key/value sequence length
    int nQHeads;    // number of query heads
    int nKVHeads;   // number of KV heads (nQH for MHA; nQH/G for GQA)
    int batch;      // batch size
    int causal;     // 1 = causal mask, 0 = full attention
};

struct DecodeCfg {
    int D;          // head dimension (64 or 128)
    int N;          // KV-cache length (number of cached keys)
    int nQHeads;    // number of query heads
    int nKVHeads;   // number of KV heads
    int batch = 1;  // new: sequences in the batch (q/o [batch][nQH][D], K/V [batch][nKVH][N][D])
};

struct DecodeDmeCfg {
    int D, N, nQHeads, nKVHeads;
    int stride_kv;  // rows between kv heads in the cache ([nKVH][stride_kv][D])
};

namespace detail {
inline cdna3_prefill_cfg to_abi(const PrefillCfg& c) {
    return cdna3_prefill_cfg{c.D, c.seqQ, c.seqK, c.nQHeads, c.nKVHeads, c.batch, c.causal};
}
inline hipError_t prefill_any(const void* Q, const void* K, const void* V, void* O, const PrefillCfg& cfg, int dtype,
                              hipStream_t stream) {
    const cdna3_prefill_cfg c = to_abi(cfg);
    return (hipError_t)cdna3_attn_prefill(Q, K, V, O, &c, dtype, (cdna4_stream_t)stream);
}
inline hipError_t decode_any(const void* q, const void* K, const void* V, void* o, const cdna3_decode_cfg& c,
                             int dtype, void* ws, size_t ws_bytes, hipStream_t stream) {
    return (hipError_t)cdna3_attn_decode(q, K, V, o, &c, dtype, ws, ws_bytes, (cdna4_stream_t)stream);
}
}  // namespace detail

// Q[batch x nQH x seqQ x D], K/V[batch x nKVH x seqK x D], O like Q.
inline hipError_t prefill(const __half* Q, const __half* K, const __half* V, __half* O, const PrefillCfg& cfg,
                          hipStream_t stream = nullptr) {
    return detail::prefill_any(Q, K, V, O, cfg, CDNA4_F16, stream);
}
inline hipError_t prefill(const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
                          __hip_bfloat16* O, const PrefillCfg& cfg, hipStream_t stream = nullptr) {
    return detail::prefill_any(Q, K, V, O, cfg, CDNA4_BF16, stream);
}
inline hipError_t prefill(const float* Q, const float* K, const float* V, float* O, const PrefillCfg& cfg,
                          hipStream_t stream = nullptr) {
    return detail::prefill_any(Q, K, V, O, cfg, CDNA4_F32, stream);
}

// q[batch x nQH x D], K/V[batch x nKVH x N x D], o[batch x nQH x D].
inline hipError_t decode(const __half* q, const __half* K, const __half* V, __half* o, const DecodeCfg& cfg,
                         hipStream_t stream = nullptr) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, cfg.batch, 0},
                              CDNA4_F16, nullptr, 0, stream);
}
inline hipError_t decode(const __hip_bfloat16* q, const __hip_bfloat16* K, const __hip_bfloat16* V,
                         __hip_bfloat16* o, const DecodeCfg& cfg, hipStream_t stream = nullptr) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, cfg.batch, 0},
                              CDNA4_BF16, nullptr, 0, stream);
}
// Caller-owned split-K workspace (>= decode_workspace_size(cfg) bytes, no initialisation).
inline size_t decode_workspace_size(const DecodeCfg& cfg) {
    const cdna3_decode_cfg c{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, cfg.batch, 0};
    return cdna3_attn_decode_workspace_size(&c);
}
inline hipError_t decode(const __half* q, const __half* K, const __half* V, __half* o, const DecodeCfg& cfg,
                         void* workspace, size_t ws_bytes, hipStream_t stream) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, cfg.batch, 0},
                              CDNA4_F16, workspace, ws_bytes, stream);
}
inline hipError_t decode(const __hip_bfloat16* q, const __hip_bfloat16* K, const __hip_bfloat16* V,
                         __hip_bfloat16* o, const DecodeCfg& cfg, void* workspace, size_t ws_bytes,
                         hipStream_t stream) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, cfg.batch, 0},
                              CDNA4_BF16, workspace, ws_bytes, stream);
}

// K/V layout [nKVHeads, stride_kv, D] head-major; pass K_layer(li, 0) as in the reference.
inline hipError_t decode_dme(const __half* q, const __half* K, const __half* V, __half* o, const DecodeDmeCfg& cfg,
                             hipStream_t stream = nullptr) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, 1, cfg.stride_kv},
                              CDNA4_F16, nullptr, 0, stream);
}
inline size_t decode_dme_workspace_size(const DecodeDmeCfg& cfg) {
    const cdna3_decode_cfg c{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, 1, cfg.stride_kv};
    return cdna3_attn_decode_workspace_size(&c);
}
inline hipError_t decode_dme(const __half* q, const __half* K, const __half* V, __half* o, const DecodeDmeCfg& cfg,
                             void* workspace, size_t ws_bytes, hipStream_t stream) {
    return detail::decode_any(q, K, V, o, cdna3_decode_cfg{cfg.D, cfg.N, cfg.nQHeads, cfg.nKVHeads, 1, cfg.stride_kv},
                              CDNA4_F16, workspace, ws_bytes, stream);
}

}  // namespace attn
}  // namespace cdna3

// The reference exposed DecodeDmeCfg at global scope (detail/fa_decode_dme_kernel.hpp:45).
using cdna3::attn::DecodeDmeCfg;
