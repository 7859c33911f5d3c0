// Drop-in check of the C++ host API: the reference's own validation program structure
// (cdna3-prims/tests/validate_attention_api.hip:77-181) written against <cdna3/attention.hpp>
// and linked to libcdna4_attn.so, with inputs and the fp32 CPU reference taken from the
// oracle (liboracle.so, loaded with dlopen). Prints one PASS/FAIL line per configuration and
// exits 0 only when all pass.
#include <cdna3/attention.hpp>
#include <cdna3/llm_integration.hpp>
#include <hip/hip_runtime.h>
#include <dlfcn.h>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef void (*fill_normal_t)(uint64_t, size_t, float, float, float*);
typedef void (*round_t)(int, const float*, size_t, float*, uint16_t*);
typedef void (*widen_t)(int, const uint16_t*, size_t, float*);
typedef int (*prefill_t)(const float*, const float*, const float*, float*, int, int, int, int, int, int, int);
typedef int (*decode_t)(const float*, const float*, const float*, float*, int, int, int, int, int, int);

static fill_normal_t fill_normal;
static round_t round_to;
static widen_t widen;
static prefill_t oracle_prefill;
static decode_t oracle_decode;

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); exit(2); } } while (0)

// |gpu - ref| <= 2e-3 * max(1, |ref|): the fp16 output's half-ulp grows with |ref|.
static bool close_enough(const std::vector<float>& got, const std::vector<float>& ref, float* worst) {
    float w = 0.f;
    for (size_t i = 0; i < got.size(); ++i) w = std::fmax(w, std::fabs(got[i] - ref[i]) / std::fmax(1.f, std::fabs(ref[i])));
    *worst = w;
    return w <= 2e-3f;
}

static bool test_prefill(int D, int seqQ, int seqK, int nQH, int nKVH, int batch, int causal, const char* label,
                         bool torch_op_launcher = false) {
    const size_t qn = (size_t)batch * nQH * seqQ * D, kn = (size_t)batch * nKVH * seqK * D;
    std::vector<float> Q(qn), K(kn), V(kn), Qr(qn), Kr(kn), Vr(kn), O(qn), Og(qn);
    std::vector<uint16_t> hQ(qn), hK(kn), hV(kn), hO(qn);
    fill_normal(42, qn, 0.f, 0.5f, Q.data());
    fill_normal(43, kn, 0.f, 0.5f, K.data());
    fill_normal(44, kn, 0.f, 0.5f, V.data());
    round_to(1, Q.data(), qn, Qr.data(), hQ.data());
    round_to(1, K.data(), kn, Kr.data(), hK.data());
    round_to(1, V.data(), kn, Vr.data(), hV.data());
    __half *dQ, *dK, *dV, *dO;
    CK(hipMalloc(&dQ, qn * 2)); CK(hipMalloc(&dK, kn * 2)); CK(hipMalloc(&dV, kn * 2)); CK(hipMalloc(&dO, qn * 2));
    CK(hipMemcpy(dQ, hQ.data(), qn * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dK, hK.data(), kn * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dV, hV.data(), kn * 2, hipMemcpyHostToDevice));
    cdna3::attn::PrefillCfg cfg{D, seqQ, seqK, nQH, nKVH, batch, causal};
    // fa_attn::launch: batch 1, causal, seqQ == seqK (the torch op's launcher)
    const hipError_t e = torch_op_launcher ? fa_attn::launch(dQ, dK, dV, dO, seqQ, nQH, nKVH, D)
                                           : cdna3::attn::prefill(dQ, dK, dV, dO, cfg);
    bool ok = false;
    float worst = 0.f;
    if (e != hipSuccess) {
        printf("  PREFILL %-36s API ERROR: %s\n", label, hipGetErrorString(e));
    } else {
        CK(hipDeviceSynchronize());
        CK(hipMemcpy(hO.data(), dO, qn * 2, hipMemcpyDeviceToHost));
        widen(1, hO.data(), qn, Og.data());
        oracle_prefill(Qr.data(), Kr.data(), Vr.data(), O.data(), D, seqQ, seqK, nQH, nKVH, batch, causal);
        ok = close_enough(Og, O, &worst);
        printf("  PREFILL %-36s err=%.6f  [%s]\n", label, worst, ok ? "PASS" : "FAIL");
    }
    CK(hipFree(dQ)); CK(hipFree(dK)); CK(hipFree(dV)); CK(hipFree(dO));
    return ok;
}

static bool test_decode(int D, int N, int nQH, int nKVH, const char* label, bool torch_op_launcher = false) {
    const size_t qn = (size_t)nQH * D, kn = (size_t)nKVH * N * D;
    std::vector<float> q(qn), K(kn), V(kn), qr(qn), Kr(kn), Vr(kn), o(qn), og(qn);
    std::vector<uint16_t> hq(qn), hK(kn), hV(kn), ho(qn);
    fill_normal(7, qn, 0.f, 0.5f, q.data());
    fill_normal(8, kn, 0.f, 0.5f, K.data());
    fill_normal(9, kn, 0.f, 0.5f, V.data());
    round_to(1, q.data(), qn, qr.data(), hq.data());
    round_to(1, K.data(), kn, Kr.data(), hK.data());
    round_to(1, V.data(), kn, Vr.data(), hV.data());
    __half *dq, *dK, *dV, *dO;
    CK(hipMalloc(&dq, qn * 2)); CK(hipMalloc(&dK, kn * 2)); CK(hipMalloc(&dV, kn * 2)); CK(hipMalloc(&dO, qn * 2));
    CK(hipMemcpy(dq, hq.data(), qn * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dK, hK.data(), kn * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dV, hV.data(), kn * 2, hipMemcpyHostToDevice));
    cdna3::attn::DecodeCfg cfg{D, N, nQH, nKVH};
    const hipError_t e = torch_op_launcher ? fa_decode::launch(dq, dK, dV, dO, fa_decode::DCfg{D, N, nQH, nKVH}, 4)
                                           : cdna3::attn::decode(dq, dK, dV, dO, cfg);
    bool ok = false;
    float worst = 0.f;
    if (e != hipSuccess) {
        printf("  DECODE  %-36s API ERROR: %s\n", label, hipGetErrorString(e));
    } else {
        CK(hipDeviceSynchronize());
        CK(hipMemcpy(ho.data(), dO, qn * 2, hipMemcpyDeviceToHost));
        widen(1, ho.data(), qn, og.data());
        oracle_decode(qr.data(), Kr.data(), Vr.data(), o.data(), D, N, nQH, nKVH, 1, 0);
        ok = close_enough(og, o, &worst);
        printf("  DECODE  %-36s err=%.6f  [%s]\n", label, worst, ok ? "PASS" : "FAIL");
    }
    CK(hipFree(dq)); CK(hipFree(dK)); CK(hipFree(dV)); CK(hipFree(dO));
    return ok;
}

int main(int argc, char** argv) {
    const char* oracle_path = argc > 1 ? argv[1] : "oracle/liboracle.so";
    void* h = dlopen(oracle_path, RTLD_NOW);
    if (!h) { printf("cannot load oracle %s: %s\n", oracle_path, dlerror()); return 2; }
    fill_normal = (fill_normal_t)dlsym(h, "orc_fill_normal_f32");
    round_to = (round_t)dlsym(h, "orc_round");
    widen = (widen_t)dlsym(h, "orc_widen");
    oracle_prefill = (prefill_t)dlsym(h, "orc_prefill_f32");
    oracle_decode = (decode_t)dlsym(h, "orc_decode_f32");
    if (!fill_normal || !round_to || !widen || !oracle_prefill || !oracle_decode) { printf("oracle symbols missing\n"); return 2; }

    int pass = 0, total = 0;
    auto chk = [&](bool r) { ++total; pass += r ? 1 : 0; };
    printf("-- Prefill (cdna3::attn::prefill) --\n");
    chk(test_prefill(128, 256, 256, 2, 2, 1, 0, "MHA full D128 seq256 h2"));
    chk(test_prefill(128, 256, 256, 4, 2, 1, 0, "GQA full D128 seq256 4q2kv"));
    chk(test_prefill(128, 256, 256, 2, 2, 1, 1, "MHA causal D128 seq256 h2"));
    chk(test_prefill(128, 256, 256, 4, 2, 1, 1, "GQA causal D128 seq256 4q2kv"));
    chk(test_prefill(64, 256, 256, 2, 2, 1, 0, "MHA full D64  seq256 h2"));
    chk(test_prefill(128, 1024, 1024, 8, 8, 1, 0, "MHA full D128 seq1024 h8"));
    chk(test_prefill(128, 512, 512, 32, 8, 1, 1, "GQA causal D128 seq512 32q8kv"));
    printf("-- Decode (cdna3::attn::decode) --\n");
    chk(test_decode(128, 128, 8, 8, "MHA D128 N128"));
    chk(test_decode(64, 128, 8, 8, "MHA D64  N128"));
    chk(test_decode(128, 512, 32, 8, "GQA D128 N512 32q8kv"));
    chk(test_decode(128, 1024, 32, 8, "GQA D128 N1024 32q8kv"));
    chk(test_decode(128, 4096, 32, 8, "GQA D128 N4096 32q8kv"));
    chk(test_decode(128, 8192, 32, 8, "GQA D128 N8192 32q8kv"));
    printf("-- torch-op launchers (fa_attn::launch, fa_decode::launch) --\n");
    chk(test_prefill(128, 256, 256, 4, 2, 1, 1, "fa_attn GQA causal D128 seq256", true));
    chk(test_prefill(64, 200, 200, 6, 6, 1, 1, "fa_attn MHA causal D64 seq200", true));
    chk(test_decode(128, 1000, 8, 2, "fa_decode GQA D128 N1000", true));
    chk(test_decode(64, 77, 4, 4, "fa_decode MHA D64 N77", true));
    printf("Result: %d/%d PASS\n", pass, total);
    return pass == total ? 0 : 1;
}
