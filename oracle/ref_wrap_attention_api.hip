// Exposes the reference's own fp32 CPU attention references (cpu_prefill, cpu_decode of
// cdna3-prims/tests/validate_attention_api.hip:27-72) through a C ABI, for pinning the oracle.
// TEST INFRASTRUCTURE ONLY: built from the reference sources in place into oracle/_ref by
// oracle/Makefile; its main() is renamed and never called, its kernels are never launched.
#include <cstring>
#define main cdna4_ref_unused_main
#include REF_SOURCE
#undef main

extern "C" int ref_cpu_prefill(const float* Q, const float* K, const float* V, float* O, int D, int seqQ, int seqK,
                               int nQH, int nKVH, int batch, int causal) {
    const size_t qn = (size_t)batch * nQH * seqQ * D, kn = (size_t)batch * nKVH * seqK * D;
    std::vector<float> q(Q, Q + qn), k(K, K + kn), v(V, V + kn), o(qn, 0.f);
    cpu_prefill(q, k, v, o, D, seqQ, seqK, nQH, nKVH, batch, causal);
    std::memcpy(O, o.data(), qn * sizeof(float));
    return 0;
}

extern "C" int ref_cpu_decode(const float* q, const float* K, const float* V, float* o, int D, int N, int nQH,
                              int nKVH) {
    const size_t qn = (size_t)nQH * D, kn = (size_t)nKVH * N * D;
    std::vector<float> qq(q, q + qn), k(K, K + kn), v(V, V + kn), oo(qn, 0.f);
    cpu_decode(qq, k, v, oo, D, N, nQH, nKVH);
    std::memcpy(o, oo.data(), qn * sizeof(float));
    return 0;
}
