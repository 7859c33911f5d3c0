// Layer-loop kernels of the small-LLM runtime (gfx950): embedding gather, fused norm + fp16 cast,
// HBM-streaming GEMVs with fused epilogues for batch-1 decode, SiLU-gated product, bias add and a
// device-side argmax.
//
// Reference behaviour restated (cdna3-prims/include/cdna3/runtime/forward.hpp): embed_gather_f32
// (:174-187), rmsnorm_f32_kernel (:34-56) followed by rocBLAS's f32 -> f16 cast
// (rocblas_gemm.hpp:36-41), the GEMM family Y = X W^T with W row-major [N][K] (:70-131,
// rocblas_gemm.hpp:8-20), silu_mul_f32 (:154-160), add_f32 (:165-168), argmax (:244-262).
//
// MI355X design: a decode step of a 768-wide model is ~111 small launches that each stream one
// weight matrix once, so every kernel here reads its weights with 16-byte loads and fuses what
// the reference ran as separate passes (norm + cast; GEMV + bias; GEMV + residual add; gate and
// up GEMVs + SiLU product). The next token id stays on the device (argmax writes it, the
// embedding gather reads it), so decode steps queue back to back without a host round trip.
// Cross-lane sums use the wave64 DPP butterfly; the only LDS is the four partial sums per row of the
// residual GEMV.
#include "common.hpp"
#include "wave_primitives/detail/xlane.hpp"
#include <math.h>

namespace cdna4 {
namespace {

using wave::xlane::allreduce;
using wave::xlane::Max;
using wave::xlane::Min;
using wave::xlane::Sum;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
__device__ __forceinline__ float dot8(const u32x4& a, const u32x4& b, float c) {
    c = dot2(a[0], b[0], c);
    c = dot2(a[1], b[1], c);
    c = dot2(a[2], b[2], c);
    return dot2(a[3], b[3], c);
}

// out[t][:] = float(embed[ids[t]][:]), one workgroup per token, 8 elements per lane step.
__global__ __launch_bounds__(256) void embed_gather(const uint16_t* __restrict__ embed, const int* __restrict__ ids,
                                                    float* __restrict__ out, int H, int V) {
    const int t = blockIdx.x;
    int id = ids[t];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    const uint16_t* src = embed + (size_t)id * H;
    float* dst = out + (size_t)t * H;
    if ((H & 7) == 0) {
        for (int c = threadIdx.x; c < H / 8; c += 256) {
            const u32x4 v = *(const u32x4*)(src + c * 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dst[c * 8 + 2 * i] = f16_bits_to_f32(v[i] & 0xffffu);
                dst[c * 8 + 2 * i + 1] = f16_bits_to_f32(v[i] >> 16);
            }
        }
    } else {
        for (int i = threadIdx.x; i < H; i += 256) dst[i] = f16_bits_to_f32(src[i]);
    }
}

// ---- a wave's share of one row ---------------------------------------------------------------
// A row of K elements (K % 8 == 0) is C = K / 8 chunks of 8; lane l holds chunks c = l + 64 j for
// j < J (zero past C). Every load is clamped to the row instead of branched around, so all of a
// lane's loads are in flight together: one memory latency per kernel, not one per chunk.
//
// Cache policy of the weight streams: a decode step reads every layer's weights once (227 MB at
// the benchmark's 12-layer d-768 model, 250 MB with its KV cache) and then the lm_head (49 MB).
// The layer weights load with the default policy and the lm_head with the non-temporal one, so
// the lm_head streams past the 256 MB Infinity Cache instead of evicting the layers, and the next
// step finds most of the layer weights there: 259.4 against 269.8 us per token with every weight
// stream non-temporal, and 268.1 with every one default (same box, interleaved).

__device__ __forceinline__ int chunk(int lane, int j, int C) { return min(lane + 64 * j, C - 1); }

template <int J, bool kStream = false>
__device__ __forceinline__ void load_f16_row(const uint16_t* __restrict__ p, int C, int lane, u32x4 (&v)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32x4* a = (const u32x4*)p + chunk(lane, j, C);
        if constexpr (kStream) v[j] = __builtin_nontemporal_load(a);
        else v[j] = *a;
    }
}

template <int J>
__device__ __forceinline__ void load_f32_row(const float* __restrict__ p, int C, int lane, f32x4 (&lo)[J],
                                             f32x4 (&hi)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const f32x4* q = (const f32x4*)p + 2 * chunk(lane, j, C);
        lo[j] = q[0];
        hi[j] = q[1];
    }
}

__device__ __forceinline__ float elem(const f32x4& lo, const f32x4& hi, int e) { return e < 4 ? lo[e] : hi[e - 4]; }
__device__ __forceinline__ float half_of(const u32x4& v, int e) {
    return f16_bits_to_f32(e & 1 ? v[e >> 1] >> 16 : v[e >> 1] & 0xffffu);
}

// Statistics of a row held as above: LayerNorm (kLayer) mean and 1/sqrt(var + eps) with var the
// mean squared deviation from the mean (two passes over the registers); RMSNorm mean 0 and
// 1/sqrt(mean(x^2) + eps). Cross-lane sums use the DPP butterfly.
template <int J, bool kLayer>
__device__ __forceinline__ void row_stats(const f32x4 (&lo)[J], const f32x4 (&hi)[J], int C, int lane, int K,
                                          float eps, float& mean, float& inv) {
    mean = 0.f;
    if constexpr (kLayer) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (lane + 64 * j < C)
#pragma unroll
                for (int e = 0; e < 8; ++e) s += elem(lo[j], hi[j], e);
        mean = allreduce(s, Sum{}) / (float)K;
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (lane + 64 * j < C)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = elem(lo[j], hi[j], e) - mean;
                q += d * d;
            }
    inv = 1.f / sqrtf(allreduce(q, Sum{}) / (float)K + eps);
}

// y = (x - mean) * inv * g (+ b) of element e of chunk j, in fp32.
template <int J>
__device__ __forceinline__ float normed(const f32x4 (&lo)[J], const f32x4 (&hi)[J], const u32x4 (&g)[J],
                                        const u32x4 (&b)[J], bool has_b, int j, int e, float mean, float inv) {
    float o = (elem(lo[j], hi[j], e) - mean) * inv * half_of(g[j], e);
    if (has_b) o += half_of(b[j], e);
    return o;
}

// Y[r][:] = norm(X[r][:]) * w + b for the prompt path, one wave per row, stored fp16 (the
// projection input). kLayer = two-pass LayerNorm, else RMSNorm.
template <int J, bool kLayer>
__global__ __launch_bounds__(256) void norm_cast(const float* __restrict__ X, const uint16_t* __restrict__ W,
                                                 const uint16_t* __restrict__ B, uint16_t* __restrict__ Y, int M,
                                                 int H, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int C = H / 8;
    f32x4 lo[J], hi[J];
    u32x4 g[J], b[J];
    load_f32_row<J>(X + (size_t)row * H, C, lane, lo, hi);
    load_f16_row<J>(W, C, lane, g);
    if (B) load_f16_row<J>(B, C, lane, b);
    float mean, inv;
    row_stats<J, kLayer>(lo, hi, C, lane, H, eps, mean, inv);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (lane + 64 * j >= C) continue;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            o[e >> 1] = f32_to_f16_bits(normed<J>(lo, hi, g, b, B != nullptr, j, e, mean, inv)) |
                        (f32_to_f16_bits(normed<J>(lo, hi, g, b, B != nullptr, j, e + 1, mean, inv)) << 16);
        *((u32x4*)(Y + (size_t)row * H) + lane + 64 * j) = o;
    }
}

// ---- decode-step GEMVs (batch 1) ---------------------------------------------------------------
// y = W x with W row-major [rows][K] fp16 and fp32 accumulation, x = a norm of the fp32 hidden row
// (each wave forms it from the row in registers). Each wave computes two rows; all W and x loads
// of the wave are issued before any arithmetic. Variants:
//   kQKV       x = norm(hidden) rounded to fp16 (the fused attention-input norm); unit u of the
//              Q block (or K, V block) takes rows d and d + D/2 of one head, so the epilogue
//              rounds y to fp16, adds the bias (rounded again, as the reference's GEMM + bias
//              kernel do), applies rotate-half RoPE at position pos to Q and K, and writes Q
//              head-major and K, V straight into the cache rows at pos
//   kSiluMul   x = norm(hidden) rounded to fp16; rows n (gate) and F + n (up):
//              act16[n] = fp16(silu(y_gate) * y_up)
//   kLogits    x = final norm(hidden) in fp32 (unrounded, as the reference's lm_head reads it);
//              rows 2u, 2u + 1: logits[r] = fp16(y) (the reference's fp16 logits store), and the
//              wave's best (value, index) key goes to the argmax partials
enum GemvKind { kQKV = 0, kSiluMul = 1, kLogits = 2 };

struct GemvArgs {
    const float* x;           // fp32 hidden row
    const uint16_t* W;
    const uint16_t* bias;     // kQKV: [QD + 2 KVD] or null
    const uint16_t* gain;     // norm weight
    const uint16_t* beta;     // norm bias or null
    float eps;
    void* out;                // kSiluMul: f16 [F]; kLogits: f32 logits [V]
    int units, K, rows;       // units = waves with work; rows = rows of W (kLogits: V)
    int pairs;                // row pairs (NP per wave)
    // kQKV
    uint16_t *q_out, *Kc, *Vc;
    const float *cos_row, *sin_row;
    int D, QD, KVD, pos, max_seq;
    // replayable step: when set, the position is *pos_dev (read on the device) and cos_row /
    // sin_row are the bases of the [max_seq][D] tables
    const int* pos_dev;
    // kLogits
    unsigned long long* partial;   // one (orderable value, ~index) key per wave
};

// Orderable 64-bit key of (value, index) that reproduces the reference's greedy choice
// (argmax_kernel, cdna3-prims/include/cdna3/runtime/forward.hpp:244-262): 256 threads each keep the
// first strict maximum of the indices t, t + 256, ..., then a tree merges thread t + s into t for
// s = 128, 64, ..., 1, keeping t on ties. Among equal values, thread t therefore wins over every
// tied thread whose index, bit-reversed over 8 bits, is larger; within a thread the smaller index
// wins. The key orders a larger value first, then the smaller (bitrev8(i % 256), i / 256), stored
// complemented in the low word.
__device__ __forceinline__ uint32_t bitrev8(uint32_t x) { return __builtin_bitreverse32(x) >> 24; }
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t ord = bitrev8((uint32_t)i & 255u) << 24 | ((uint32_t)i >> 8);
    return ((unsigned long long)u << 32) | (uint32_t)(0xffffffffu - ord);
}
__device__ __forceinline__ int argmax_index(uint32_t low_word) {
    const uint32_t ord = 0xffffffffu - low_word;
    return (int)((ord & 0xffffffu) * 256u + bitrev8(ord >> 24));
}

// Rows (r0, r1) of row pair p of a GEMV kind (see above).
template <int kKind>
__device__ __forceinline__ void pair_rows(const GemvArgs& a, int p, int& r0, int& r1) {
    if constexpr (kKind == kQKV) {
        const int half = a.D / 2;
        int base = 0, u = p;
        if (u >= a.QD / 2 + a.KVD / 2) { base = a.QD + a.KVD; u -= a.QD / 2 + a.KVD / 2; }
        else if (u >= a.QD / 2) { base = a.QD; u -= a.QD / 2; }
        r0 = base + (u / half) * a.D + u % half;
        r1 = r0 + half;
    } else if constexpr (kKind == kSiluMul) {
        r0 = p;
        r1 = p + a.rows / 2;
    } else {
        r0 = 2 * p;
        r1 = min(2 * p + 1, a.rows - 1);
    }
}

// Each wave takes NP consecutive row pairs, so the norm of the hidden row (loaded, reduced and
// formed in every wave) is paid once per 2 NP rows.
template <int kKind, int J, bool kLayer, int NP>
__global__ __launch_bounds__(256) void gemv2(GemvArgs a) {
    const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (unit >= a.units) return;
    const int K = a.K, C = K / 8;
    int r0[NP], r1[NP];
    u32x4 w0[NP][J], w1[NP][J];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        pair_rows<kKind>(a, min(unit * NP + p, a.pairs - 1), r0[p], r1[p]);
        load_f16_row<J, kKind == 2>(a.W + (size_t)r0[p] * K, C, lane, w0[p]);   // lm_head: streamed
        load_f16_row<J, kKind == 2>(a.W + (size_t)r1[p] * K, C, lane, w1[p]);
    }
    float y0[NP], y1[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) y0[p] = y1[p] = 0.f;
    {
        f32x4 lo[J], hi[J];
        u32x4 g[J], b[J];
        load_f32_row<J>(a.x, C, lane, lo, hi);
        load_f16_row<J>(a.gain, C, lane, g);
        if (a.beta) load_f16_row<J>(a.beta, C, lane, b);
        float mean, inv;
        row_stats<J, kLayer>(lo, hi, C, lane, K, a.eps, mean, inv);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if (lane + 64 * j >= C) continue;
            if constexpr (kKind == kLogits) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xe = normed<J>(lo, hi, g, b, a.beta != nullptr, j, e, mean, inv);
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        y0[p] = fmaf(half_of(w0[p][j], e), xe, y0[p]);
                        y1[p] = fmaf(half_of(w1[p][j], e), xe, y1[p]);
                    }
                }
            } else {
                u32x4 xn;
#pragma unroll
                for (int e = 0; e < 8; e += 2)
                    xn[e >> 1] = f32_to_f16_bits(normed<J>(lo, hi, g, b, a.beta != nullptr, j, e, mean, inv)) |
                                 (f32_to_f16_bits(normed<J>(lo, hi, g, b, a.beta != nullptr, j, e + 1, mean, inv))
                                  << 16);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    y0[p] = dot8(w0[p][j], xn, y0[p]);
                    y1[p] = dot8(w1[p][j], xn, y1[p]);
                }
            }
        }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        y0[p] = allreduce(y0[p], Sum{});
        y1[p] = allreduce(y1[p], Sum{});
    }
    if (lane != 0) return;   // every lane holds the sums: lane 0 stores
    if constexpr (kKind == kLogits) {
        float* lg = (float*)a.out;
        unsigned long long best = 0ull;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if (unit * NP + p >= a.pairs) continue;
            // The reference stores the logits as fp16 (gemm_f32in_f16out_kernel) and takes the
            // argmax of those values.
            const float v0 = (float)(_Float16)y0[p], v1 = (float)(_Float16)y1[p];
            lg[r0[p]] = v0;
            if (r1[p] != r0[p]) lg[r1[p]] = v1;
            const unsigned long long k0 = argmax_key(v0, r0[p]), k1 = argmax_key(v1, r1[p]);
            const unsigned long long k = k0 > k1 ? k0 : k1;
            best = k > best ? k : best;
        }
        a.partial[unit] = best;   // the wave's best (value, index) key for the argmax
        return;
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if (unit * NP + p >= a.pairs) continue;
        const float ya = y0[p], yb = y1[p];
        const int ra = r0[p], rb = r1[p];
        if constexpr (kKind == kSiluMul) {
            ((uint16_t*)a.out)[ra] = (uint16_t)f32_to_f16_bits(ya / (1.f + expf(-ya)) * yb);
        } else {   // kQKV
            uint32_t h0 = f32_to_f16_bits(ya), h1 = f32_to_f16_bits(yb);
            if (a.bias) {
                h0 = f32_to_f16_bits(f16_bits_to_f32(h0) + f16_bits_to_f32(a.bias[ra]));
                h1 = f32_to_f16_bits(f16_bits_to_f32(h1) + f16_bits_to_f32(a.bias[rb]));
            }
            const int half = a.D / 2;
            int pos = a.pos;
            const float *cos_row = a.cos_row, *sin_row = a.sin_row;
            if (a.pos_dev) {
                pos = *a.pos_dev;
                cos_row += (size_t)pos * a.D;
                sin_row += (size_t)pos * a.D;
            }
            if (ra < a.QD + a.KVD) {   // Q or K: rotate the pair (d, d + D/2)
                const int d = (ra % a.D);
                const float t0 = f16_bits_to_f32(h0), t1 = f16_bits_to_f32(h1);
                h0 = f32_to_f16_bits(t0 * cos_row[d] - t1 * sin_row[d]);
                h1 = f32_to_f16_bits(t1 * cos_row[d + half] + t0 * sin_row[d + half]);
            }
            if (ra < a.QD) {
                a.q_out[ra] = (uint16_t)h0;
                a.q_out[rb] = (uint16_t)h1;
            } else {
                const bool is_k = ra < a.QD + a.KVD;
                const int rr = ra - (is_k ? a.QD : a.QD + a.KVD);
                uint16_t* cache = (is_k ? a.Kc : a.Vc) + ((size_t)(rr / a.D) * a.max_seq + pos) * a.D + rr % a.D;
                cache[0] = (uint16_t)h0;
                cache[half] = (uint16_t)h1;
            }
        }
    }
}

// out32[r] += W[r][:] . x for fp16 x (the O and down projections of a decode step): one workgroup
// per row, the row's 16-byte chunks split over its four waves (wave w: chunks q0 + l + 64 j of its
// quarter, lane l), so a 768-row GEMV still spreads over every CU instead of the 96 workgroups of
// two rows per wave (measured +3.6 % tokens/s for the config-5 decode step over that form). The
// four partial sums meet in LDS and are added in wave order. All loads are issued before any
// arithmetic.
constexpr int kSplitWaves = 4;

template <int J>
__global__ __launch_bounds__(64 * kSplitWaves) void gemv_residual_split(const uint16_t* __restrict__ x,
                                                                        const uint16_t* __restrict__ W,
                                                                        float* __restrict__ out, int K) {
    __shared__ float part[kSplitWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int C = K / 8, Q = (C + kSplitWaves - 1) / kSplitWaves;   // chunks per row, per wave
    const int q0 = wave * Q, qn = min(C, q0 + Q) - q0;              // this wave's chunks (qn may be <= 0)
    const int row = blockIdx.x;
    u32x4 w[J], xv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {   // loads clamped into the row, masked below
        const int c = min(q0 + min(lane + 64 * j, max(qn - 1, 0)), C - 1);
        xv[j] = ((const u32x4*)x)[c];
        w[j] = ((const u32x4*)(W + (size_t)row * K))[c];
    }
    float y = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (lane + 64 * j < qn) y = dot8(w[j], xv[j], y);
    y = allreduce(y, Sum{});
    if (lane == 0) part[wave] = y;
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = part[0];
#pragma unroll
        for (int i = 1; i < kSplitWaves; ++i) acc += part[i];
        out[row] += acc;
    }
}

// The attention output x (fp16, [heads][D] flat, K = heads * D) merged from the split-K partials
// of the decode attention: chunk c of x (8 elements of head h = 8c / D) is
// fp16(sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p), M = max_p m_p, over the P (<= kMaxParts)
// partials part_ml[(h P + p) * 2] = (m_p, l_p), part_o[(h P + p) D + d] (the layout the decode
// kernels write, batch 1). Rounded once, as the decode kernels round o.
constexpr int kMaxParts = 4;

__device__ __forceinline__ u32x4 merged_chunk(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                              int P, int D, int c) {
    const int h = (8 * c) / D, d0 = (8 * c) % D;
    float2 ml[kMaxParts];
    float4 lo[kMaxParts], hi[kMaxParts];
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {   // every load issued before any arithmetic
        const int pp = min(p, P - 1);
        ml[p] = *(const float2*)(part_ml + ((size_t)h * P + pp) * 2);
        lo[p] = *(const float4*)(part_o + ((size_t)h * P + pp) * D + d0);
        hi[p] = *(const float4*)(part_o + ((size_t)h * P + pp) * D + d0 + 4);
    }
    float M = ml[0].x;
#pragma unroll
    for (int p = 1; p < kMaxParts; ++p)
        if (p < P) M = fmaxf(M, ml[p].x);
    float L = 0.f, v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
        if (p >= P) break;
        const float wt = exp2f(ml[p].x - M);
        L = fmaf(wt, ml[p].y, L);
        v[0] = fmaf(wt, lo[p].x, v[0]); v[1] = fmaf(wt, lo[p].y, v[1]);
        v[2] = fmaf(wt, lo[p].z, v[2]); v[3] = fmaf(wt, lo[p].w, v[3]);
        v[4] = fmaf(wt, hi[p].x, v[4]); v[5] = fmaf(wt, hi[p].y, v[5]);
        v[6] = fmaf(wt, hi[p].z, v[6]); v[7] = fmaf(wt, hi[p].w, v[7]);
    }
    const float inv = L > 0.f ? 1.f / L : 1.f;
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = f32_to_f16_bits(v[2 * i] * inv) | (f32_to_f16_bits(v[2 * i + 1] * inv) << 16);
    return r;
}

// gemv_residual_split with its input vector merged from decode partials (merged_chunk).
template <int J>
__global__ __launch_bounds__(64 * kSplitWaves) void gemv_residual_merge(const float* __restrict__ part_ml,
                                                                        const float* __restrict__ part_o, int P, int D,
                                                                        const uint16_t* __restrict__ W,
                                                                        float* __restrict__ out, int K) {
    __shared__ float part[kSplitWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int C = K / 8, Q = (C + kSplitWaves - 1) / kSplitWaves;
    const int q0 = wave * Q, qn = min(C, q0 + Q) - q0;
    const int row = blockIdx.x;
    u32x4 w[J], xv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = min(q0 + min(lane + 64 * j, max(qn - 1, 0)), C - 1);
        w[j] = ((const u32x4*)(W + (size_t)row * K))[c];
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = min(q0 + min(lane + 64 * j, max(qn - 1, 0)), C - 1);
        xv[j] = merged_chunk(part_ml, part_o, P, D, c);
    }
    float y = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (lane + 64 * j < qn) y = dot8(w[j], xv[j], y);
    y = allreduce(y, Sum{});
    if (lane == 0) part[wave] = y;
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = part[0];
#pragma unroll
        for (int i = 1; i < kSplitWaves; ++i) acc += part[i];
        out[row] += acc;
    }
}

// Final argmax over the per-wave keys of the logits GEMV: one workgroup of 1024 lanes, each
// folding a strided share (loads issued 8 at a time), then the DPP butterfly per wave and wave 0
// over the 16 wave results. Writes the token to ids[0] and tokens[step] and, when embed is
// given, the token's embedding row to next_row (the next decode step's input). With a device step state {pos, step} (replayable steps), step is read from it
// and both fields advance by one, ready for the next replay.
__global__ __launch_bounds__(1024) void argmax_keys(const unsigned long long* __restrict__ keys, int n,
                                                    unsigned long long* __restrict__ scratch, int* __restrict__ ids,
                                                    int* __restrict__ tokens, int step, int* __restrict__ state,
                                                    const uint16_t* __restrict__ embed, float* __restrict__ next_row,
                                                    int H, int V) {
    unsigned long long best = 0;
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * 1024) {
        unsigned long long k[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) k[u] = (i0 + u * 1024 < n) ? keys[i0 + u * 1024] : 0ull;
#pragma unroll
        for (int u = 0; u < 8; ++u) best = k[u] > best ? k[u] : best;
    }
    // wave max of 64-bit keys: high word first, then the low word among lanes holding that high word
    uint32_t hi = (uint32_t)(best >> 32), lo = (uint32_t)best;
    const uint32_t mhi = (uint32_t)allreduce((int)(hi ^ 0x80000000u), Max{}) ^ 0x80000000u;
    const uint32_t mlo = (uint32_t)allreduce((int)((hi == mhi ? lo : 0u) ^ 0x80000000u), Max{}) ^ 0x80000000u;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = ((unsigned long long)mhi << 32) | mlo;
    __syncthreads();
    // Every wave folds the 16 wave maxima itself, so the winner needs no broadcast.
    {
        const unsigned lane = threadIdx.x & 63;
        const unsigned long long k = lane < 16 ? scratch[lane] : 0ull;
        hi = (uint32_t)(k >> 32);
        lo = (uint32_t)k;
    }
    const uint32_t h2 = (uint32_t)allreduce((int)(hi ^ 0x80000000u), Max{}) ^ 0x80000000u;
    const uint32_t l2 = (uint32_t)allreduce((int)((hi == h2 ? lo : 0u) ^ 0x80000000u), Max{}) ^ 0x80000000u;
    const int tok = argmax_index(l2);
    if (threadIdx.x == 0) {
        ids[0] = tok;
        if (state) step = state[1];
        if (tokens) tokens[step] = tok;
        if (state) {
            state[0] += 1;
            state[1] = step + 1;
        }
    }
    // The next step's input: the chosen token's embedding row as fp32 (H % 8 == 0), so the step
    // needs no separate gather launch.
    if (!embed) return;
    const int id = min(max(tok, 0), V - 1);
    const uint16_t* src = embed + (size_t)id * H;
    for (int c = threadIdx.x; c < H / 8; c += 1024) {
        const u32x4 v = *(const u32x4*)(src + c * 8);
        f32x4 lo, hi;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            lo[2 * i] = f16_bits_to_f32(v[i] & 0xffffu);
            lo[2 * i + 1] = f16_bits_to_f32(v[i] >> 16);
            hi[2 * i] = f16_bits_to_f32(v[i + 2] & 0xffffu);
            hi[2 * i + 1] = f16_bits_to_f32(v[i + 2] >> 16);
        }
        *(f32x4*)(next_row + c * 8) = lo;
        *(f32x4*)(next_row + c * 8 + 4) = hi;
    }
}

// act[t][n] = fp16(silu(gu[t][n]) * gu[t][F + n]) for the prompt path (gu fp32 [T][2F]).
__global__ __launch_bounds__(256) void silu_mul(const float* __restrict__ gu, uint16_t* __restrict__ act, int T,
                                                int F) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * F) return;
    const size_t t = i / F, n = i % F;
    const float g = gu[t * 2 * F + n], u = gu[t * 2 * F + F + n];
    act[i] = (uint16_t)f32_to_f16_bits(g / (1.f + expf(-g)) * u);
}

// Y[t][n] = fp16(Y[t][n] + b[n]) (QKV bias after the prompt GEMM).
__global__ __launch_bounds__(256) void bias_add_f16(uint16_t* __restrict__ Y, const uint16_t* __restrict__ b, int T,
                                                    int N) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * N) return;
    Y[i] = (uint16_t)f32_to_f16_bits(f16_bits_to_f32(Y[i]) + f16_bits_to_f32(b[i % N]));
}

}  // namespace

// ---- host-side launchers used by the runtime (csrc/session.hip) ---------------------------

int llm_embed(const void* embed, const int* ids, float* out, int T, int H, int V, hipStream_t s) {
    embed_gather<<<T, 256, 0, s>>>((const uint16_t*)embed, ids, out, H, V);
    return launch_status();
}

namespace {
// Smallest supported chunk count per lane for a row of K elements (K % 8 == 0; K <= 4096, or
// K <= 8192 for the fp16-input GEMV).
int chunks_per_lane(int K) {
    const int j = (K / 8 + 63) / 64;
    return j <= 1 ? 1 : j <= 2 ? 2 : j <= 3 ? 3 : j <= 4 ? 4 : j <= 6 ? 6 : j <= 8 ? 8 : j <= 12 ? 12 : j <= 16 ? 16 : 0;
}

template <int J>
void norm_cast_launch(bool layer, const float* X, const void* W, const void* B, void* Y, int M, int H, float eps,
                      hipStream_t s) {
    const unsigned grid = ceil_div(M, 4);
    if (layer)
        norm_cast<J, true><<<grid, 256, 0, s>>>(X, (const uint16_t*)W, (const uint16_t*)B, (uint16_t*)Y, M, H, eps);
    else
        norm_cast<J, false><<<grid, 256, 0, s>>>(X, (const uint16_t*)W, (const uint16_t*)B, (uint16_t*)Y, M, H, eps);
}

// Row pairs per wave of each kind. The lm_head GEMV (32,000 rows at config 5) has parallelism to
// spare and gains from paying its norm once per 8 rows (+1 % tokens/s); the Q/K/V and gate/up
// GEMVs measured slower with two pairs per wave (fewer waves in flight).
constexpr int kPairsQKV = 1, kPairsSilu = 1, kPairsLogits = 4;
template <int kKind> constexpr int pairs_per_wave() {
    return kKind == kQKV ? kPairsQKV : (kKind == kSiluMul ? kPairsSilu : kPairsLogits);
}

template <int kKind, int J>
void gemv_launch(bool layer, GemvArgs a, hipStream_t s) {
    constexpr int NP = pairs_per_wave<kKind>();
    a.units = (a.pairs + NP - 1) / NP;
    const unsigned grid = ceil_div(a.units, 4);
    if (layer) gemv2<kKind, J, true, NP><<<grid, 256, 0, s>>>(a);
    else gemv2<kKind, J, false, NP><<<grid, 256, 0, s>>>(a);
}

template <int kKind>
int gemv_dispatch(bool layer, const GemvArgs& a, hipStream_t s) {
    switch (chunks_per_lane(a.K)) {
        case 1: gemv_launch<kKind, 1>(layer, a, s); break;
        case 2: gemv_launch<kKind, 2>(layer, a, s); break;
        case 3: gemv_launch<kKind, 3>(layer, a, s); break;
        case 4: gemv_launch<kKind, 4>(layer, a, s); break;
        case 6: gemv_launch<kKind, 6>(layer, a, s); break;
        case 8: gemv_launch<kKind, 8>(layer, a, s); break;
        default: return CDNA4_ERR_INVALID_VALUE;
    }
    return launch_status();
}

// Norm-fused kinds hold the fp32 row in registers: K <= 4096. The fp16-input GEMV: K <= 8192.
bool gemv_shape_ok(int K, bool fp16_input = false) {
    return K >= 8 && K % 8 == 0 && K <= (fp16_input ? 8192 : 4096);
}
}  // namespace

int llm_norm_cast(bool layer, const float* X, const void* W, const void* B, void* Y, int M, int H, float eps,
                  hipStream_t s) {
    if (!gemv_shape_ok(H)) return CDNA4_ERR_INVALID_VALUE;
    switch (chunks_per_lane(H)) {
        case 1: norm_cast_launch<1>(layer, X, W, B, Y, M, H, eps, s); break;
        case 2: norm_cast_launch<2>(layer, X, W, B, Y, M, H, eps, s); break;
        case 3: norm_cast_launch<3>(layer, X, W, B, Y, M, H, eps, s); break;
        case 4: norm_cast_launch<4>(layer, X, W, B, Y, M, H, eps, s); break;
        case 6: norm_cast_launch<6>(layer, X, W, B, Y, M, H, eps, s); break;
        default: norm_cast_launch<8>(layer, X, W, B, Y, M, H, eps, s); break;
    }
    return launch_status();
}

// out[n] += W[n] . x with x merged from P decode partials of K / D heads (batch 1; see merged_chunk).
int llm_gemv_residual_merge(const float* part_ml, const float* part_o, int P, int D, const void* W, float* out, int N,
                            int K, hipStream_t s) {
    if (!gemv_shape_ok(K, true) || N < 1 || P < 1 || P > kMaxParts || D % 8 || K % D) return CDNA4_ERR_INVALID_VALUE;
    const int q = (K / 8 + kSplitWaves - 1) / kSplitWaves;
    const uint16_t* WW = (const uint16_t*)W;
    const unsigned grid = (unsigned)N, block = 64 * kSplitWaves;
    switch ((q + 63) / 64) {
        case 1: gemv_residual_merge<1><<<grid, block, 0, s>>>(part_ml, part_o, P, D, WW, out, K); break;
        case 2: gemv_residual_merge<2><<<grid, block, 0, s>>>(part_ml, part_o, P, D, WW, out, K); break;
        case 3: gemv_residual_merge<3><<<grid, block, 0, s>>>(part_ml, part_o, P, D, WW, out, K); break;
        default: gemv_residual_merge<4><<<grid, block, 0, s>>>(part_ml, part_o, P, D, WW, out, K); break;
    }
    return launch_status();
}

int llm_gemv_residual(const void* x, const void* W, float* out, int N, int K, hipStream_t s) {
    if (!gemv_shape_ok(K, true) || N < 1) return CDNA4_ERR_INVALID_VALUE;
    const int q = (K / 8 + kSplitWaves - 1) / kSplitWaves;   // chunks per wave: at most 256 (K <= 8192)
    const uint16_t *xx = (const uint16_t*)x, *WW = (const uint16_t*)W;
    const unsigned grid = (unsigned)N, block = 64 * kSplitWaves;
    switch ((q + 63) / 64) {
        case 1: gemv_residual_split<1><<<grid, block, 0, s>>>(xx, WW, out, K); break;
        case 2: gemv_residual_split<2><<<grid, block, 0, s>>>(xx, WW, out, K); break;
        case 3: gemv_residual_split<3><<<grid, block, 0, s>>>(xx, WW, out, K); break;
        default: gemv_residual_split<4><<<grid, block, 0, s>>>(xx, WW, out, K); break;
    }
    return launch_status();
}

int llm_gemv_qkv(bool layer, const float* hidden, const void* gain, const void* beta, float eps, const void* W,
                 const void* bias, int H, int D, int nH, int nKV, const float* cos_row, const float* sin_row,
                 void* q_out, void* Kc, void* Vc, int pos, int max_seq, hipStream_t s, const int* pos_dev) {
    if (!gemv_shape_ok(H) || D % 2) return CDNA4_ERR_INVALID_VALUE;
    GemvArgs a{};
    a.x = hidden; a.W = (const uint16_t*)W; a.bias = (const uint16_t*)bias; a.gain = (const uint16_t*)gain;
    a.beta = (const uint16_t*)beta; a.eps = eps; a.K = H;
    a.D = D; a.QD = nH * D; a.KVD = nKV * D; a.rows = a.QD + 2 * a.KVD; a.pairs = a.rows / 2;
    a.cos_row = cos_row; a.sin_row = sin_row; a.q_out = (uint16_t*)q_out; a.Kc = (uint16_t*)Kc;
    a.Vc = (uint16_t*)Vc; a.pos = pos; a.max_seq = max_seq; a.pos_dev = pos_dev;
    return gemv_dispatch<kQKV>(layer, a, s);
}

int llm_gemv_silu(bool layer, const float* hidden, const void* gain, const void* beta, float eps, const void* W,
                  void* act, int F, int H, hipStream_t s) {
    if (!gemv_shape_ok(H) || F < 1) return CDNA4_ERR_INVALID_VALUE;
    GemvArgs a{};
    a.x = hidden; a.W = (const uint16_t*)W; a.gain = (const uint16_t*)gain; a.beta = (const uint16_t*)beta;
    a.eps = eps; a.out = act; a.K = H; a.rows = 2 * F; a.pairs = F;
    return gemv_dispatch<kSiluMul>(layer, a, s);
}

// Argmax partial keys of the logits GEMV for a vocabulary of V (one per wave; an upper bound).
size_t llm_argmax_partials(int V) { return (size_t)(V + 1) / 2; }

int llm_logits_argmax(bool layer, const float* hidden, const void* gain, const void* beta, float eps,
                      const void* W, float* logits, int V, int H, unsigned long long* partial,
                      unsigned long long* scratch16, int* ids, int* tokens, int step, hipStream_t s, int* state,
                      const void* embed, float* next_row) {
    if (!gemv_shape_ok(H) || V < 1) return CDNA4_ERR_INVALID_VALUE;
    GemvArgs a{};
    a.x = hidden; a.W = (const uint16_t*)W; a.gain = (const uint16_t*)gain; a.beta = (const uint16_t*)beta;
    a.eps = eps; a.out = logits; a.K = H; a.rows = V; a.pairs = (V + 1) / 2; a.partial = partial;
    if (int e = gemv_dispatch<kLogits>(layer, a, s)) return e;
    constexpr int NP = pairs_per_wave<kLogits>();
    argmax_keys<<<1, 1024, 0, s>>>(partial, (a.pairs + NP - 1) / NP, scratch16, ids, tokens, step, state,
                                   (const uint16_t*)embed, next_row, H, V);
    return launch_status();
}

namespace {
__global__ void step_state(int* state, int pos, int step) {
    if (threadIdx.x == 0) {
        state[0] = pos;
        state[1] = step;
    }
}
}  // namespace

// Device step state {pos, step} of replayed decode steps.
int llm_step_state(int* state, int pos, int step, hipStream_t s) {
    step_state<<<1, 64, 0, s>>>(state, pos, step);
    return launch_status();
}

int llm_silu_mul(const float* gu, void* act, int T, int F, hipStream_t s) {
    silu_mul<<<ceil_div((size_t)T * F, 256), 256, 0, s>>>(gu, (uint16_t*)act, T, F);
    return launch_status();
}

int llm_bias_add_f16(void* Y, const void* b, int T, int N, hipStream_t s) {
    bias_add_f16<<<ceil_div((size_t)T * N, 256), 256, 0, s>>>((uint16_t*)Y, (const uint16_t*)b, T, N);
    return launch_status();
}

}  // namespace cdna4
