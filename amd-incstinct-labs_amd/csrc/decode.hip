// Split-K flash decode for gfx950: one query token per sequence, GQA, fp16/bf16 KV cache.
//
// Reference behaviour restated (cdna3-prims/include/cdna3/detail/fa_decode_kernel.hpp:21-94,
// fa_decode_dme_kernel.hpp:64-208, launched by attention.hpp:117-173): o = softmax(q K^T /
// sqrt(D)) V per query head, query head h reading kv head h / (nQH / nKVH), fp32 softmax and
// accumulation.
//
// MI355X design (not the reference's structure):
//   * Each wave streams its own contiguous range of keys of one (batch, kv head) and
//     serves every query head of the GQA group from registers, so K/V bytes are read from
//     HBM exactly once (the reference re-reads a kv head once per query head).
//   * A key row is D*2 bytes = D/8 lanes x 16 bytes: every load is a fully coalesced 128-bit
//     global load, 64 lanes cover 64*16 bytes of consecutive keys, U loads of K and of V are
//     in flight per lane.
//   * q.k uses v_dot2_f32_{f16,bf16} (fp32 accumulation), the per-key lane-group sum is the
//     DPP row butterfly; softmax runs in base 2 with a log2(e)-prescaled scale.
//   * Each wave merges its lane groups with the permlane swaps and writes one (m, l, O)
//     partial per query head; a second kernel merges the partials of each query head, with
//     the max and the denominator formed by the wave butterfly. No LDS is used anywhere.
#include "common.hpp"
#include "wave_primitives/detail/xlane.hpp"
#include <mutex>
#include <math.h>

namespace cdna4 {
namespace {

using wave::xlane::allreduce;
using wave::xlane::cross_row_allreduce;
using wave::xlane::dpp_full;
using wave::xlane::Sum;
using wave::xlane::Max;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));

constexpr int kDecodeU = 4;           // keys per lane group per iteration (loads in flight)
constexpr int kDecodeWaves = 4;       // independent waves per 256-thread workgroup
constexpr int kTargetWaves = 4096;    // 16 waves per CU on 256 CUs
constexpr int kMaxHeadsPerWave = 8;   // query heads served from one pass over K/V
constexpr float kLog2e = 1.4426950408889634f;

template <bool kBf16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (kBf16) return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, a), __builtin_bit_cast(b2_t, b), c, false);
    else return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
template <bool kBf16>
__device__ __forceinline__ void unpack8(const u32x4& v, float (&o)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (kBf16) { o[2 * i] = bf16_bits_to_f32(v[i] & 0xffffu); o[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16); }
        else { o[2 * i] = f16_bits_to_f32(v[i] & 0xffffu); o[2 * i + 1] = f16_bits_to_f32(v[i] >> 16); }
    }
}
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (kBf16) return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
    else return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

// Sum over the D/8 lanes that share one key row (16 lanes at D=128, 8 at D=64).
template <int D>
__device__ __forceinline__ float keyrow_sum(float v) {
    v += dpp_full<wave::xlane::kQuadXor1>(v);
    v += dpp_full<wave::xlane::kQuadXor2>(v);
    v += dpp_full<wave::xlane::kRowHalfMirror>(v);
    if constexpr (D == 128) v += dpp_full<wave::xlane::kRowMirror>(v);
    return v;
}

// Combine the per-lane-group values of one lane position over all lane groups of the wave.
template <int D, class Op>
__device__ __forceinline__ float across_groups(float v, Op op) {
    if constexpr (D == 64) v = op(v, dpp_full<0x128>(v));   // row_ror:8 pairs the two 8-lane groups of a row
    return cross_row_allreduce(v, op);
}

struct DecodeArgs {
    const void* q; const void* K; const void* V;
    float* part_ml;   // [batch][nQH][P][2]
    float* part_o;    // [batch][nQH][P][D]
    int N, nQH, nKVH, stride, G, HB, KPW, P;
    float sc;         // log2(e) / sqrt(D)
};

template <int D, int HB, bool kBf16>
__global__ __launch_bounds__(256) void decode_partial(DecodeArgs a) {
    constexpr int LPK = D / 8;            // lanes per key row
    constexpr int KPL = 64 / LPK;         // key rows per wave load
    const unsigned lane = threadIdx.x & 63u;
    const int wave_split = blockIdx.x * kDecodeWaves + (int)(threadIdx.x >> 6);
    if (wave_split >= a.P) return;
    const int kvh = blockIdx.y / (a.G / HB);
    const int sub = blockIdx.y % (a.G / HB);
    const int b = blockIdx.z;
    const int qh0 = kvh * a.G + sub * HB;
    const int row = (int)lane / LPK, c = (int)lane % LPK;

    const int kbeg = wave_split * a.KPW;
    const int kend = min(a.N, kbeg + a.KPW);
    const size_t head_off = ((size_t)b * a.nKVH + kvh) * (size_t)a.stride * D;
    const uint16_t* Kh = (const uint16_t*)a.K + head_off + c * 8;
    const uint16_t* Vh = (const uint16_t*)a.V + head_off + c * 8;

    u32x4 q[HB];
#pragma unroll
    for (int h = 0; h < HB; ++h)
        q[h] = *(const u32x4*)((const uint16_t*)a.q + ((size_t)b * a.nQH + qh0 + h) * D + c * 8);

    float m[HB], l[HB], o[HB][8];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
        m[h] = -INFINITY; l[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
    }

    for (int k0 = kbeg; k0 < kend; k0 += KPL * kDecodeU) {
        u32x4 kv[kDecodeU], vv[kDecodeU];
        bool valid[kDecodeU];
#pragma unroll
        for (int j = 0; j < kDecodeU; ++j) {
            const int key = k0 + row + KPL * j;
            valid[j] = key < kend;
            const int kk = valid[j] ? key : kbeg;     // in-bounds address for masked rows
            kv[j] = __builtin_nontemporal_load((const u32x4*)(Kh + (size_t)kk * D));
            vv[j] = __builtin_nontemporal_load((const u32x4*)(Vh + (size_t)kk * D));
        }
        float s[kDecodeU][HB];
#pragma unroll
        for (int j = 0; j < kDecodeU; ++j) {
#pragma unroll
            for (int h = 0; h < HB; ++h) {
                float t = dot2<kBf16>(q[h][0], kv[j][0], 0.f);
                t = dot2<kBf16>(q[h][1], kv[j][1], t);
                t = dot2<kBf16>(q[h][2], kv[j][2], t);
                t = dot2<kBf16>(q[h][3], kv[j][3], t);
                t = keyrow_sum<D>(t);
                s[j][h] = valid[j] ? t * a.sc : -INFINITY;
            }
        }
        float vf[kDecodeU][8];
#pragma unroll
        for (int j = 0; j < kDecodeU; ++j) unpack8<kBf16>(vv[j], vf[j]);
#pragma unroll
        for (int h = 0; h < HB; ++h) {
            float mx = s[0][h];
#pragma unroll
            for (int j = 1; j < kDecodeU; ++j) mx = fmaxf(mx, s[j][h]);
            const float mnew = fmaxf(m[h], mx);
            const float mref = (mnew == -INFINITY) ? 0.f : mnew;
            const float alpha = exp2f(m[h] - mref);
            float p[kDecodeU], ps = 0.f;
#pragma unroll
            for (int j = 0; j < kDecodeU; ++j) { p[j] = exp2f(s[j][h] - mref); ps += p[j]; }
            l[h] = l[h] * alpha + ps;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float acc = o[h][e] * alpha;
#pragma unroll
                for (int j = 0; j < kDecodeU; ++j) acc = fmaf(p[j], vf[j][e], acc);
                o[h][e] = acc;
            }
            m[h] = mnew;
        }
    }

    // Merge the lane groups of this wave, then lane group 0 writes the wave's partial.
#pragma unroll
    for (int h = 0; h < HB; ++h) {
        const float M = across_groups<D>(m[h], Max{});
        const float w = (M == -INFINITY) ? 0.f : exp2f(m[h] - M);
        const float L = across_groups<D>(l[h] * w, Sum{});
        float ov[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ov[e] = across_groups<D>(o[h][e] * w, Sum{});
        const size_t pidx = ((size_t)b * a.nQH + qh0 + h) * a.P + wave_split;
        if (row == 0) {
            float4* dst = (float4*)(a.part_o + pidx * D + c * 8);
            dst[0] = make_float4(ov[0], ov[1], ov[2], ov[3]);
            dst[1] = make_float4(ov[4], ov[5], ov[6], ov[7]);
            if (c == 0) *(float2*)(a.part_ml + pidx * 2) = make_float2(M, L);
        }
    }
}

// One wave per (batch, query head): o = sum_i 2^(m_i - M) O_i / sum_i 2^(m_i - M) l_i.
template <int D, bool kBf16>
__global__ __launch_bounds__(64) void decode_merge(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                                   void* __restrict__ out, int P) {
    constexpr int EPL = D / 64;
    const unsigned lane = threadIdx.x;
    const size_t bh = blockIdx.x;
    const float* ml = part_ml + bh * P * 2;
    const float* po = part_o + bh * P * D;
    float M = -INFINITY;
    for (int i = lane; i < P; i += 64) M = fmaxf(M, ml[2 * i]);
    M = allreduce(M, Max{});
    const float Mref = (M == -INFINITY) ? 0.f : M;
    float L = 0.f;
    for (int i = lane; i < P; i += 64) L += ml[2 * i + 1] * exp2f(ml[2 * i] - Mref);
    L = allreduce(L, Sum{});
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
    for (int i = 0; i < P; ++i) {
        const float w = exp2f(ml[2 * i] - Mref);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(w, po[(size_t)i * D + lane * EPL + e], acc[e]);
    }
    const float inv = (L > 0.f) ? 1.f / L : 1.f;
    uint16_t* o = (uint16_t*)out + bh * D + lane * EPL;
    if constexpr (EPL == 2) {
        *(uint32_t*)o = pack2<kBf16>(acc[0] * inv, acc[1] * inv);
    } else {
        o[0] = (uint16_t)(kBf16 ? f32_to_bf16_bits(acc[0] * inv) : f32_to_f16_bits(acc[0] * inv));
    }
}

struct Plan { int G, HB, subgroups, KPW, P; size_t ws_bytes; };

bool plan_decode(const cdna3_decode_cfg& c, Plan& p) {
    if (c.D != 64 && c.D != 128) return false;
    if (c.N < 1 || c.nQHeads < 1 || c.nKVHeads < 1 || c.batch < 1) return false;
    if (c.nQHeads % c.nKVHeads) return false;
    const int stride = c.stride_kv == 0 ? c.N : c.stride_kv;
    if (stride < c.N) return false;
    p.G = c.nQHeads / c.nKVHeads;
    p.HB = 1;
    for (int hb = kMaxHeadsPerWave; hb >= 1; --hb)
        if (p.G % hb == 0) { p.HB = hb; break; }
    p.subgroups = p.G / p.HB;
    const int kpl = 64 / (c.D / 8);
    const int step = kpl * kDecodeU;
    const double rows = (double)c.batch * c.nKVHeads * p.subgroups;
    long long kpw = (long long)ceil((double)c.N * rows / kTargetWaves);
    if (kpw < 2 * step) kpw = 2 * step;
    kpw = (kpw + step - 1) / step * step;
    if (kpw > c.N) kpw = ((long long)c.N + step - 1) / step * step;
    p.KPW = (int)kpw;
    p.P = (int)((c.N + kpw - 1) / kpw);
    p.ws_bytes = (size_t)c.batch * c.nQHeads * p.P * (size_t)(c.D + 2) * sizeof(float) + 256;
    return true;
}

template <int D, bool kBf16>
int launch_decode(const cdna3_decode_cfg& c, const Plan& p, const void* q, const void* K, const void* V, void* o,
                  void* ws, hipStream_t s) {
    DecodeArgs a;
    a.q = q; a.K = K; a.V = V;
    const size_t nml = (size_t)c.batch * c.nQHeads * p.P * 2;
    a.part_ml = (float*)ws;
    a.part_o = (float*)((char*)ws + ((nml * sizeof(float) + 255) & ~(size_t)255));
    a.N = c.N; a.nQH = c.nQHeads; a.nKVH = c.nKVHeads; a.stride = c.stride_kv == 0 ? c.N : c.stride_kv;
    a.G = p.G; a.HB = p.HB; a.KPW = p.KPW; a.P = p.P;
    a.sc = kLog2e / sqrtf((float)D);
    dim3 grid(ceil_div(p.P, kDecodeWaves), c.nKVHeads * p.subgroups, c.batch);
    switch (p.HB) {
        case 1: decode_partial<D, 1, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 2: decode_partial<D, 2, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 3: decode_partial<D, 3, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 4: decode_partial<D, 4, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 5: decode_partial<D, 5, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 6: decode_partial<D, 6, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 7: decode_partial<D, 7, kBf16><<<grid, 256, 0, s>>>(a); break;
        case 8: decode_partial<D, 8, kBf16><<<grid, 256, 0, s>>>(a); break;
        default: return CDNA4_ERR_INVALID_VALUE;
    }
    decode_merge<D, kBf16><<<(unsigned)((size_t)c.batch * c.nQHeads), 64, 0, s>>>(a.part_ml, a.part_o, o, p.P);
    return launch_status();
}

// Per-device fallback workspace for callers that pass none (the reference launchers take
// no workspace argument). Grown on demand, kept until process exit.
struct FallbackWs { std::mutex mu; void* ptr[64] = {}; size_t bytes[64] = {}; };
FallbackWs g_ws;

int fallback_workspace(size_t need, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return CDNA4_ERR_INVALID_VALUE;
    std::lock_guard<std::mutex> lk(g_ws.mu);
    if (g_ws.bytes[dev] < need) {
        // The old buffer may still be read by queued work on another stream: leak it
        // rather than free it under that work. Growth is geometric, so this is bounded.
        size_t sz = g_ws.bytes[dev] ? g_ws.bytes[dev] * 2 : (size_t)1 << 20;
        while (sz < need) sz *= 2;
        void* p = nullptr;
        e = hipMalloc(&p, sz);
        if (e != hipSuccess) return (int)e;
        g_ws.ptr[dev] = p;
        g_ws.bytes[dev] = sz;
    }
    *out = g_ws.ptr[dev];
    return 0;
}

}  // namespace
}  // namespace cdna4

using namespace cdna4;

extern "C" size_t cdna3_attn_decode_workspace_size(const cdna3_decode_cfg* cfg) {
    Plan p;
    if (!cfg || !plan_decode(*cfg, p)) return 0;
    return p.ws_bytes + 256;
}

extern "C" int cdna3_attn_decode(const void* q, const void* K, const void* V, void* o, const cdna3_decode_cfg* cfg,
                                 int dtype, void* workspace, size_t ws_bytes, cdna4_stream_t stream) {
    Plan p;
    if (!cfg || !plan_decode(*cfg, p)) return CDNA4_ERR_INVALID_VALUE;
    if (dtype != CDNA4_F16 && dtype != CDNA4_BF16) return CDNA4_ERR_INVALID_VALUE;
    if (!q || !K || !V || !o) return CDNA4_ERR_INVALID_VALUE;
    // 16-byte loads of q/K/V rows.
    if ((((uintptr_t)q | (uintptr_t)K | (uintptr_t)V) & 15u) != 0) return CDNA4_ERR_INVALID_VALUE;
    if (((uintptr_t)o & 3u) != 0) return CDNA4_ERR_INVALID_VALUE;
    const size_t need = p.ws_bytes + 256;
    if (workspace != nullptr && ws_bytes < need) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    if (workspace == nullptr) {
        if (int e = fallback_workspace(need, &workspace)) return e;
    }
    hipStream_t s = (hipStream_t)stream;
    const bool bf = dtype == CDNA4_BF16;
    if (cfg->D == 128) return bf ? launch_decode<128, true>(*cfg, p, q, K, V, o, workspace, s)
                                 : launch_decode<128, false>(*cfg, p, q, K, V, o, workspace, s);
    return bf ? launch_decode<64, true>(*cfg, p, q, K, V, o, workspace, s)
              : launch_decode<64, false>(*cfg, p, q, K, V, o, workspace, s);
}
