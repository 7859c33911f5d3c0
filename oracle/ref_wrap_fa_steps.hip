// Exposes the reference's fp32 CPU reference of the FA2 reference configuration (attn_cpu_ref,
// research/flash-attention-mi300x/fa_naive.hip:217-243) through a C ABI, for pinning the oracle.
// TEST INFRASTRUCTURE ONLY: built in place from the reference sources into oracle/_ref by
// oracle/Makefile; its main() is renamed and never called, its kernels are never launched.
#include <cstring>
#define main cdna4_ref_unused_main
#include REF_SOURCE
#undef main

// One (batch, head) slice: Q [seq_q][d], K and V [seq_k][d].
extern "C" int ref_attn_cpu_ref(const float* Q, const float* K, const float* V, float* O, int seq_q, int seq_k,
                                int d) {
    std::vector<float> q(Q, Q + (size_t)seq_q * d), k(K, K + (size_t)seq_k * d), v(V, V + (size_t)seq_k * d);
    std::vector<float> o((size_t)seq_q * d, 0.f);
    attn_cpu_ref(q, k, v, o, seq_q, seq_k, d);
    std::memcpy(O, o.data(), o.size() * sizeof(float));
    return 0;
}
