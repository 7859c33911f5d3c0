#pragma once
// cdna3/runtime/kv_cache.hpp — contiguous fp16 KV cache for batch-1 decode (gfx950 build).
//
// Same type, fields and members as the reference's KVCache (cdna3-prims/include/cdna3/runtime/
// kv_cache.hpp:19-52): K and V are [n_layers][n_kv_heads][max_seq_len][head_dim] fp16, the layout
// cdna3::attn::decode_dme reads in place (stride_kv = max_seq_len) and cdna3_attn_prefill_strided
// reads for the prompt. K_layer(layer, pos) / V_layer(layer, pos) point at kv head 0, token pos of a
// layer. Differences: allocate() returns the HIP error instead of dropping it (and leaves K, V null
// on failure), and the byte count is computed in size_t throughout. Host code only; include with any
// C++ compiler that sees the HIP runtime headers.
#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include <stddef.h>

namespace cdna3 {
namespace runtime {

struct KVCache {
    __half* K = nullptr;   // device: [n_layers x n_kv_heads x max_seq_len x head_dim]
    __half* V = nullptr;
    int n_layers = 0;
    int n_kv_heads = 0;
    int max_seq_len = 0;
    int head_dim = 0;
    int len = 0;           // tokens currently stored

    size_t bytes() const { return (size_t)n_layers * n_kv_heads * max_seq_len * head_dim * sizeof(__half); }

    hipError_t allocate(int nl, int nkvh, int max_seq, int hdim) {
        free_buffers();
        n_layers = nl;
        n_kv_heads = nkvh;
        max_seq_len = max_seq;
        head_dim = hdim;
        len = 0;
        const size_t b = bytes();
        hipError_t e = hipMalloc((void**)&K, b);
        if (e == hipSuccess) e = hipMalloc((void**)&V, b);
        if (e == hipSuccess) e = hipMemset(K, 0, b);
        if (e == hipSuccess) e = hipMemset(V, 0, b);
        if (e != hipSuccess) free_buffers();
        return e;
    }

    void free_buffers() {
        if (K) (void)hipFree(K);
        if (V) (void)hipFree(V);
        K = V = nullptr;
    }

    __half* K_layer(int layer, int pos = 0) const {
        return K + ((size_t)layer * n_kv_heads * max_seq_len + pos) * head_dim;
    }
    __half* V_layer(int layer, int pos = 0) const {
        return V + ((size_t)layer * n_kv_heads * max_seq_len + pos) * head_dim;
    }
};

}  // namespace runtime
}  // namespace cdna3
