#pragma once
// cdna3/llm_integration.hpp — the launchers behind the reference's PyTorch ops, host side (gfx950).
//
// Drop-in for research/flash-attention-mi300x/llm_integration/fa_attn_kernel.hpp:141-150
// (fa_attn::launch) and fa_decode_kernel.hpp:20, :103-113 (fa_decode::DCfg, fa_decode::launch),
// over libcdna4_attn.so. Same names, arguments, layouts and return type:
//   fa_attn::launch(Q, K, V, O, seq, nQH, nKVH, D, stream)    causal GQA prefill, head-major
//                                                              Q, O [nQH][seq][D], K, V [nKVH][seq][D]
//   fa_decode::launch(q, K, V, o, DCfg{D, N, nQH, nKVH}, W, stream)
//                                                              one query per head, q, o [nQH][D],
//                                                              K, V [nKVH][N][D]
// Differences: any seq >= 1 is computed (the reference required seq % 16 == 0 and dropped the
// tail otherwise); W, the reference's split-KV wave count (2 or 4), is validated as there but the
// library chooses its own plan; decode runs the one-launch plan that needs no workspace (no
// allocation, nothing shared between calls), as the reference's launcher did. That plan runs one
// workgroup per (kv head, group of 16 query heads): 8 CUs for 32 q / 8 kv heads, 74 us at N 8192
// (D 128, fp16) on one MI355X. Callers decoding a few long sequences should call
// cdna3::attn::decode with a workspace (<cdna3/attention.hpp>), 11-14 us at that shape.
#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include "../cdna4_attn.h"

namespace fa_attn {

inline hipError_t launch(const __half* Q, const __half* K, const __half* V, __half* O, int seq, int nQH, int nKVH,
                         int D, hipStream_t stream = 0) {
    const cdna3_prefill_cfg c{D, seq, seq, nQH, nKVH, 1, 1};
    return (hipError_t)cdna3_attn_prefill(Q, K, V, O, &c, CDNA4_F16, (cdna4_stream_t)stream);
}

}  // namespace fa_attn

namespace fa_decode {

struct DCfg { int D, N, nQHeads, nKVHeads; };

inline hipError_t launch(const __half* q, const __half* K, const __half* V, __half* o, DCfg c, int W,
                         hipStream_t stream = 0) {
    if (W != 2 && W != 4) return hipErrorInvalidValue;
    const cdna3_decode_cfg d{c.D, c.N, c.nQHeads, c.nKVHeads, 1, 0};
    return (hipError_t)cdna3_attn_decode(q, K, V, o, &d, CDNA4_F16, nullptr, 0, (cdna4_stream_t)stream);
}

}  // namespace fa_decode
