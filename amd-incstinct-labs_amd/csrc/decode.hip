// Split-K flash decode for gfx950: one query token per sequence, GQA, fp16/bf16 KV cache.
//
// Reference behaviour restated (cdna3-prims/include/cdna3/detail/fa_decode_kernel.hpp:21-94,
// fa_decode_dme_kernel.hpp:64-208, launched by attention.hpp:117-173): o = softmax(q K^T /
// sqrt(D)) V per query head, query head h reading kv head h / (nQH / nKVH), fp32 softmax and
// accumulation.
//
// MI355X design (not the reference's structure):
//   * Split-K: each single-wave workgroup streams one contiguous range of keys of one (batch,
//     kv head) and serves all query heads of the GQA group (up to 16 per wave) at once, so K/V
//     bytes are read from HBM exactly once (the reference re-reads a kv head once per query
//     head). The q.K and P.V products run on the matrix cores with the prefill tile machinery
//     (the heads take the place of the 16 query columns), which leaves the VALU only the
//     softmax: the kernel is bound by HBM, not by per-element dot products.
//   * K/V chunks go HBM -> LDS by asynchronous global_load_lds copies into a ring of stages,
//     three chunks per wave in flight. The split-K kernel's copies carry the non-temporal policy
//     (every K/V byte is read once): config 4 measured 5.8 -> 6.6 TB/s with it, with the
//     Infinity Cache holding other data. The one-launch kernel takes it for caches larger than
//     the Infinity Cache only: the runtime's decode step, whose caches are small and just
//     appended to, ran 3 % slower with it.
//   * When batch x kv heads fills whole rounds of the CUs (config 4: 256 on 256), one workgroup
//     per (batch, kv head) streams its whole cache and merges its waves in LDS: no split-K
//     partials, no merge launch (159.8 us against 162.6 us for split + merge at config 4).
//   * A second kernel merges the (m, l, O) partials of each query head, with the max and the
//     denominator formed by the wave butterfly.
#include "attn_tile.hpp"
#include "attn_stream.hpp"
#include <atomic>
#include <math.h>

namespace cdna4 {
namespace {

using namespace stream;

using wave::xlane::allreduce;
using wave::xlane::Sum;
using wave::xlane::Max;
using tile::f32x4;

constexpr float kLog2e = 1.4426950408889634f;

template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (kBf16) return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
    else return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

struct DecodeArgs {
    const void* q; const void* K; const void* V;
    float* part_ml;   // [batch][nQH][P][2]
    float* part_o;    // [batch][nQH][P][D]
    int N, nQH, nKVH, stride, G, HB, KPW, P;   // HB: groups of <= 16 query heads per kv head
    float sc;         // log2(e) / sqrt(D)
    // Replayable launches (a captured decode step): when set, the cache length is *len_pos + 1,
    // read on the device, and the short-cache variant sizes its per-wave key ranges from it.
    const int* len_pos;
};

// ---- matrix-core split-K partial -----------------------------------------------------------
//
// One single-wave workgroup per (key split, batch, kv head, group of up to 16 query heads). The
// query heads of the GQA group are the 16 "query" columns of the prefill tile machinery
// (S^T = K Q^T, O^T = V^T P^T on 16x16x32 MFMAs, lazy base-2 softmax), so each K/V byte is
// read from HBM once for all heads of its group, and the per-byte VALU work is the softmax of
// 16 columns instead of a dot product per element. Keys stream in 32-key chunks through a ring
// of NS LDS stages filled by asynchronous global->LDS copies (16 bytes per lane, no VGPRs): the
// copy of chunk c + NS - 1 is issued before chunk c is computed, so NS - 1 chunks per wave are
// in flight while the matrix cores work. A single wave needs no barrier: it waits (vmcnt) for
// its own copies, and a stage is refilled only after the wave's reads of it have completed.
constexpr int kDecPerCU = 4;    // resident single-wave workgroups per CU the grid is sized for

// Query heads of the group as B operands: lane holds q[head qh0 + li][32c + 8g .. +8], zero
// past the group.
template <int D>
__device__ __forceinline__ void load_q(const DecodeArgs& a, int b, int qh0, int nrows, int li, int g,
                                       u32x4 (&qb)[1][D / 32]) {
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
        qb[0][c] = u32x4{0u, 0u, 0u, 0u};
        if (li < nrows)
            qb[0][c] = *(const u32x4*)((const uint16_t*)a.q + ((size_t)b * a.nQH + qh0 + li) * D + c * 32 + g * 8);
        asm volatile("" : : "v"(qb[0][c]));   // the loads complete before the first copy is issued
    }
}

template <int D, bool kBf16, int NS>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void decode_mfma(DecodeArgs a) {
    static_assert(NS >= 2 && NS <= 4, "ring depth");
    constexpr int ND = D / 32, NDT = D / 16;
    constexpr int kStage = kDecT * D;                 // elements per K (or V) stage
    constexpr int kCopies = 2 * kDecT * (D / 8) / 64;  // copies per stage (K and V)
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[NS * kStage];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[NS * kStage];

    const int lane = (int)threadIdx.x;
    const int li = lane & 15, g = lane >> 4;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.HB;                // HB = head groups of 16 per kv head
    const int sub = blockIdx.y % a.HB;
    const int b = blockIdx.z;
    const int qh0 = kvh * a.G + sub * 16;
    const int nrows = min(16, a.G - sub * 16);

    const int N = a.len_pos ? *a.len_pos + 1 : a.N;
    const int kbeg = split * a.KPW;
    const int kend = min(N, kbeg + a.KPW);
    const int nch = (kend - kbeg + kDecT - 1) / kDecT;
    const size_t head_off = ((size_t)b * a.nKVH + kvh) * (size_t)a.stride * D;
    const uint16_t* Kh = (const uint16_t*)a.K + head_off;
    const uint16_t* Vh = (const uint16_t*)a.V + head_off;

    // Query heads as B operands: lane holds q[head qh0 + li][32c + 8g .. +8], zero past the group.
    u32x4 qb[1][ND];
#pragma unroll
    for (int c = 0; c < ND; ++c) {
        qb[0][c] = u32x4{0u, 0u, 0u, 0u};
        if (li < nrows)
            qb[0][c] = *(const u32x4*)((const uint16_t*)a.q + ((size_t)b * a.nQH + qh0 + li) * D + c * 32 + g * 8);
        asm volatile("" : : "v"(qb[0][c]));   // the loads complete before the first copy is issued
    }
    f32x4 o[1][NDT], lacc[1];
    float m[1] = {tile::kInitM};
    lacc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[0][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const tile::LdsOffsets off = tile::lds_offsets<D>(li, g);

#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < nch) {
            load_stage<D, true, true>(Kh, D, kbeg + i * kDecT, N, k_lds + i * kStage, lane);
            load_stage<D, false, true>(Vh, D, kbeg + i * kDecT, N, v_lds + i * kStage, lane);
        }
    int st = 0;   // stage of chunk ch
    for (int ch = 0; ch < nch; ++ch) {
        const int ahead = ch + NS - 1;
        if (ahead < nch) {
            const int sa = (st == 0) ? NS - 1 : st - 1;   // stage of chunk ch - 1, already consumed
            load_stage<D, true, true>(Kh, D, kbeg + ahead * kDecT, N, k_lds + sa * kStage, lane);
            load_stage<D, false, true>(Vh, D, kbeg + ahead * kDecT, N, v_lds + sa * kStage, lane);
        }
        wait_copies_younger<kCopies>(min(NS - 1, nch - 1 - ch));
        const char* Kt = (const char*)(k_lds + st * kStage);
        const char* Vt = (const char*)(v_lds + st * kStage);
        const int kb = kbeg + ch * kDecT;
        f32x4 s[1][2];
        tile::qk_chunk<D, 1, kBf16>(Kt, off, qb, s, 0);
        float lm[1];
        const bool need = (kb + kDecT > kend)
            ? tile::check_chunk<1, true>(s, m, lm, kb, 0, kend, 0, a.sc, li, g)
            : tile::check_chunk<1, false>(s, m, lm, kb, 0, kend, 0, a.sc, li, g);
        if (__builtin_amdgcn_ballot_w64(need)) tile::rescale_rows<D, 1>(lm, m, o, lacc, a.sc);
        u32x4 pb[1];
        tile::softmax_chunk<1, kBf16>(s, m, pb, a.sc);
        tile::pv_chunk<D, 1, kBf16>(Vt, off, pb, o, lacc, 0);
        if constexpr (kBf16) {
            if (kb < tile::kLoKeys) {   // the first keys of the cache: the weights' second bf16 term
                tile::softmax_lo_chunk<1>(s, m, pb, a.sc);
                tile::pv_chunk<D, 1, true>(Vt, off, pb, o, lacc, 0);
            }
        }
        st = (st == NS - 1) ? 0 : st + 1;
    }

    // Partial (m, l, O) of each head of the group: lane holds O^T[16dt + 4g + e][head li].
    if (li < nrows) {
        const size_t pidx = ((size_t)b * a.nQH + qh0 + li) * a.P + split;
        float* dst = a.part_o + pidx * D + g * 4;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            *(float4*)(dst + dt * 16) = make_float4(o[0][dt][0], o[0][dt][1], o[0][dt][2], o[0][dt][3]);
        if (g == 0) *(float2*)(a.part_ml + pidx * 2) = make_float2(m[0], lacc[0][0]);
    }
}

// ---- short caches: one launch, split-K inside the workgroup --------------------------------
//
// For short caches the split-K grid above is small and its second (merge) launch costs as much
// as the attention itself. Here one workgroup of W waves serves a (batch, kv head, head group):
// wave w streams the w-th of W contiguous key ranges through its own LDS ring, then the waves
// leave their (m, l, O) partials in LDS (over their rings, after a barrier) and all W*64 lanes
// merge them, o = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w, writing the output directly.
template <int D, int W>
constexpr int wg_ring_elems() { return W * kDecStages * kDecT * D; }

// Keys per wave of the short-cache variant: N split into W ranges of whole 32-key chunks.
__host__ __device__ constexpr int wg_keys_per_wave(int N, int W) { return ((N + W - 1) / W + kDecT - 1) / kDecT * kDecT; }

// Keys per workgroup when the cache is split over P workgroups per (batch, kv head, head group):
// N in P ranges of whole 32-key chunks.
__host__ __device__ constexpr int wg_keys_per_split(int N, int P) { return ((N + P - 1) / P + kDecT - 1) / kDecT * kDecT; }

// kNT: the copies take the non-temporal policy (long caches; see plan_decode).
// kPart: workgroup blockIdx.x of a.P serves the blockIdx.x-th of P key ranges (wg_keys_per_split)
// and leaves the merged (m, l, O) of its waves in the split-K partials (a.part_ml, a.part_o)
// instead of writing o; a consumer merges the P partials of each query head.
template <int D, bool kBf16, int W, bool kNT, bool kPart = false>
__global__ __launch_bounds__(64 * W) void decode_wg(DecodeArgs a, void* __restrict__ out) {
    constexpr int ND = D / 32, NDT = D / 16;
    constexpr int kStage = kDecT * D;
    constexpr int kRing = kDecStages * kStage;
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[wg_ring_elems<D, W>()];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[wg_ring_elems<D, W>()];
    static_assert((size_t)W * 16 * D * sizeof(float) <= sizeof(k_lds), "O partials fit over the K rings");
    static_assert((size_t)W * 16 * 2 * sizeof(float) <= sizeof(v_lds), "(m, l) partials fit over the V rings");

    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const int li = lane & 15, g = lane >> 4;
    const int kvh = blockIdx.y / a.HB;
    const int sub = blockIdx.y % a.HB;
    const int b = blockIdx.z;
    const int qh0 = kvh * a.G + sub * 16;
    const int nrows = min(16, a.G - sub * 16);
    const int N = a.len_pos ? *a.len_pos + 1 : a.N;
    int s0 = 0, s1 = N;   // this workgroup's keys
    if constexpr (kPart) {
        const int KPS = wg_keys_per_split(N, a.P);
        s0 = min(N, (int)blockIdx.x * KPS);
        s1 = min(N, s0 + KPS);
    }
    const int KPW = (a.len_pos || kPart) ? wg_keys_per_wave(s1 - s0, W) : a.KPW;
    const int kbeg = min(s1, s0 + wave * KPW);
    const int kend = min(s1, kbeg + KPW);
    const size_t head_off = ((size_t)b * a.nKVH + kvh) * (size_t)a.stride * D;

    u32x4 qb[1][ND];
    load_q<D>(a, b, qh0, nrows, li, g, qb);
    f32x4 o[1][NDT], lacc[1];
    float m[1];
    stream_keys<D, kBf16, kDecStages, kNT>((const uint16_t*)a.K + head_off, (const uint16_t*)a.V + head_off, D, N, kbeg,
                                      kend, 0, 0, a.sc, qb, o, lacc, m, k_lds + wave * kRing, v_lds + wave * kRing,
                                      lane);
    if constexpr (kPart)
        merge_waves_part<D, W>(o, lacc, m, (float*)k_lds, (float*)v_lds, nrows, a.part_ml, a.part_o,
                               (size_t)b * a.nQH + qh0, a.P, (int)blockIdx.x, wave, lane);
    else
        merge_waves<D, kBf16, W>(o, lacc, m, (float*)k_lds, (float*)v_lds, nrows,
                                 (uint16_t*)out + ((size_t)b * a.nQH + qh0) * D, wave, lane);
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
    // Up to 64 partials per pass: lane j computes partial j's weight once (0 for lanes past the
    // count) and the loop takes it back with v_readlane (no LDS). Sixteen partials' rows are loaded
    // before any is used; indices past the count re-read the last row, weighted 0.
    for (int i0 = 0; i0 < P; i0 += 64) {
        const int n = min(64, P - i0);
        const float wl = ((int)lane < n) ? exp2f(ml[2 * (i0 + (int)lane)] - Mref) : 0.f;
        const float* pi = po + (size_t)i0 * D + lane * EPL;
        for (int j0 = 0; j0 < n; j0 += 16) {   // j0 <= 48, so j0 + jj <= 63 below
            float v[16][EPL];
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const int j = min(j0 + jj, n - 1);
#pragma unroll
                for (int e = 0; e < EPL; ++e) v[jj][e] = pi[(size_t)j * D + e];
            }
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j0 + jj));
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[e] = fmaf(w, v[jj][e], acc[e]);
            }
        }
    }
    const float inv = (L > 0.f) ? 1.f / L : 1.f;
    uint16_t* o = (uint16_t*)out + bh * D + lane * EPL;
    if constexpr (EPL == 2) {
        *(uint32_t*)o = pack2<kBf16>(acc[0] * inv, acc[1] * inv);
    } else {
        o[0] = (uint16_t)(kBf16 ? f32_to_bf16_bits(acc[0] * inv) : f32_to_f16_bits(acc[0] * inv));
    }
}

// The merge for P <= NR partials: every load (each partial's (m, l) on lane p, and all NR rows)
// issued before any arithmetic, so the merge costs one memory round trip instead of one for the
// (m, l) values and one per sixteen rows. Same arithmetic and order as decode_merge (bit-identical).
template <int D, bool kBf16, int NR>
__global__ __launch_bounds__(64) void decode_merge_short(const float* __restrict__ part_ml,
                                                         const float* __restrict__ part_o, void* __restrict__ out,
                                                         int P) {
    constexpr int EPL = D / 64;
    static_assert(NR <= 64, "one partial per lane");
    const unsigned lane = threadIdx.x;
    const size_t bh = blockIdx.x;
    const float* ml = part_ml + bh * P * 2;
    const float* pi = part_o + bh * P * D + lane * EPL;
    const bool has = (int)lane < P;
    const float mi = has ? ml[2 * lane] : -INFINITY;
    const float li = has ? ml[2 * lane + 1] : 0.f;
    float v[NR][EPL];   // rows past P re-read row P - 1 and are weighted 0
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[j][e] = pi[(size_t)min(j, P - 1) * D + e];
    const float M = allreduce(mi, Max{});
    const float Mref = (M == -INFINITY) ? 0.f : M;
    const float wl = has ? exp2f(mi - Mref) : 0.f;
    const float L = allreduce(has ? li * exp2f(mi - Mref) : 0.f, Sum{});
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j));
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(w, v[j][e], acc[e]);
    }
    const float inv = (L > 0.f) ? 1.f / L : 1.f;
    uint16_t* o = (uint16_t*)out + bh * D + lane * EPL;
    if constexpr (EPL == 2) {
        *(uint32_t*)o = pack2<kBf16>(acc[0] * inv, acc[1] * inv);
    } else {
        o[0] = (uint16_t)(kBf16 ? f32_to_bf16_bits(acc[0] * inv) : f32_to_f16_bits(acc[0] * inv));
    }
}

struct Plan { int G, HB, KPW, P; size_t ws_bytes; bool wg, nt; };

// Waves per workgroup of the short-cache variant (its LDS holds W rings of two K and V stages)
// and the longest cache it takes when a split-K workspace is available: at most kWgChunks 32-key
// chunks per wave.
template <int D> constexpr int wg_waves() { return D == 64 ? 8 : 4; }
constexpr int kWgChunks = 8;

// HB: groups of up to 16 query heads per kv head (one MFMA column block each); KPW: keys per
// split, a multiple of the 32-key chunk, sized so that the whole grid is one round of resident
// workgroups (kDecPerCU per CU): every workgroup streams from start to end with no second round
// and no tail of stragglers, which measured markedly faster than many short splits.
// split_k == false (a call without a workspace) always takes the one-launch variant, which needs
// no memory beyond q, K, V and o: such a call never allocates and shares no buffer with any other
// call, so it is re-entrant across streams and capturable. Long caches then stream through one
// workgroup per (batch, kv head, head group) instead of a split-K grid.
// With a workspace, long caches also take the one-launch variant when its grid is whole rounds of
// one workgroup per CU (batch x kv heads x head groups a multiple of the CU count): every CU then
// streams the same number of rows from start to end, as the split grid's workgroups do, and the
// call skips the merge launch and the partials (config 4, 256 rows on 256 CUs: 159.8 us against
// 162.6 us for split + merge, both with non-temporal copies).
// nt: K/V larger than the 256 MB Infinity Cache are copied with the non-temporal policy (no call
// can find them cached anyway); smaller caches, such as the runtime's per-layer caches, keep the
// default policy (the runtime's decode step measured 3 % slower with non-temporal copies).
constexpr double kStreamBytes = 256.0 * 1024 * 1024;

// CDNA4_DECODE_SPLIT_K=1 in the environment (read on every call, including the workspace-size and
// plan queries) keeps calls with a workspace on the split-K plan where whole rounds of CUs would
// otherwise take the one-launch plan, so the two plans can be timed against each other.
bool force_split_k() {
    const char* e = getenv("CDNA4_DECODE_SPLIT_K");
    return e && e[0] == '1';
}

bool plan_decode(const cdna3_decode_cfg& c, bool split_k, Plan& p) {
    if (c.D != 64 && c.D != 128) return false;
    if (c.N < 1 || c.nQHeads < 1 || c.nKVHeads < 1 || c.batch < 1) return false;
    if (c.nQHeads % c.nKVHeads) return false;
    const int stride = c.stride_kv == 0 ? c.N : c.stride_kv;
    if (stride < c.N) return false;
    p.G = c.nQHeads / c.nKVHeads;
    p.HB = (p.G + 15) / 16;
    const int W = c.D == 64 ? wg_waves<64>() : wg_waves<128>();
    const long long rows = (long long)c.batch * c.nKVHeads * p.HB;
    const int cus = device_cus();
    p.nt = 4.0 * c.batch * c.nKVHeads * (double)c.N * c.D > kStreamBytes;
    p.wg = !split_k || c.N <= W * kWgChunks * kDecT || (cus > 0 && rows % cus == 0 && !force_split_k());
    if (p.wg) {   // one workgroup per (batch, kv head, head group); W contiguous key ranges
        p.KPW = wg_keys_per_wave(c.N, W);
        p.P = 1;
        p.ws_bytes = 0;
        return true;
    }
    const double slots = (double)cus * kDecPerCU;
    long long kpw = (long long)ceil((double)c.N * (double)rows / slots);
    if (kpw < 4 * kDecT) kpw = 4 * kDecT;
    kpw = (kpw + kDecT - 1) / kDecT * kDecT;
    if (kpw > c.N) kpw = ((long long)c.N + kDecT - 1) / kDecT * kDecT;
    p.KPW = (int)kpw;
    p.P = (int)((c.N + kpw - 1) / kpw);
    if (p.P > 65535) return false;
    p.ws_bytes = (size_t)c.batch * c.nQHeads * p.P * (size_t)(c.D + 2) * sizeof(float) + 256;
    return true;
}

template <int D, bool kBf16>
int launch_decode(const cdna3_decode_cfg& c, const Plan& p, const void* q, const void* K, const void* V, void* o,
                  void* ws, hipStream_t s, const int* len_pos = nullptr) {
    DecodeArgs a;
    a.len_pos = len_pos;
    a.q = q; a.K = K; a.V = V;
    const size_t nml = (size_t)c.batch * c.nQHeads * p.P * 2;
    a.part_ml = (float*)ws;
    a.part_o = ws ? (float*)((char*)ws + ((nml * sizeof(float) + 255) & ~(size_t)255)) : nullptr;
    a.N = c.N; a.nQH = c.nQHeads; a.nKVH = c.nKVHeads; a.stride = c.stride_kv == 0 ? c.N : c.stride_kv;
    a.G = p.G; a.HB = p.HB; a.KPW = p.KPW; a.P = p.P;
    a.sc = kLog2e / sqrtf((float)D);
    const long long gy = (long long)c.nKVHeads * p.HB;
    if (gy > 65535 || c.batch > 65535) return CDNA4_ERR_INVALID_VALUE;
    dim3 grid((unsigned)p.P, (unsigned)gy, (unsigned)c.batch);
    if (p.wg) {
        if (p.nt) decode_wg<D, kBf16, wg_waves<D>(), true><<<grid, 64 * wg_waves<D>(), 0, s>>>(a, o);
        else decode_wg<D, kBf16, wg_waves<D>(), false><<<grid, 64 * wg_waves<D>(), 0, s>>>(a, o);
        return launch_status();
    }
    if (!ws) return CDNA4_ERR_INVALID_VALUE;
    decode_mfma<D, kBf16, kDecStages><<<grid, 64, 0, s>>>(a);
    const unsigned nbh = (unsigned)((size_t)c.batch * c.nQHeads);
    if (p.P <= 16) decode_merge_short<D, kBf16, 16><<<nbh, 64, 0, s>>>(a.part_ml, a.part_o, o, p.P);
    else if (p.P <= 64) decode_merge_short<D, kBf16, 64><<<nbh, 64, 0, s>>>(a.part_ml, a.part_o, o, p.P);
    else decode_merge<D, kBf16><<<nbh, 64, 0, s>>>(a.part_ml, a.part_o, o, p.P);
    return launch_status();
}

int check_decode_args(const void* q, const void* K, const void* V, void* o, int dtype) {
    if (dtype != CDNA4_F16 && dtype != CDNA4_BF16) return CDNA4_ERR_INVALID_VALUE;
    if (!q || !K || !V || !o) return CDNA4_ERR_INVALID_VALUE;
    // 16-byte loads of q/K/V rows.
    if ((((uintptr_t)q | (uintptr_t)K | (uintptr_t)V) & 15u) != 0) return CDNA4_ERR_INVALID_VALUE;
    if (((uintptr_t)o & 3u) != 0) return CDNA4_ERR_INVALID_VALUE;
    return 0;
}

int run_decode(const cdna3_decode_cfg& c, const Plan& p, const void* q, const void* K, const void* V, void* o,
               int dtype, void* ws, hipStream_t s) {
    const bool bf = dtype == CDNA4_BF16;
    if (c.D == 128) return bf ? launch_decode<128, true>(c, p, q, K, V, o, ws, s)
                              : launch_decode<128, false>(c, p, q, K, V, o, ws, s);
    return bf ? launch_decode<64, true>(c, p, q, K, V, o, ws, s) : launch_decode<64, false>(c, p, q, K, V, o, ws, s);
}

// ---- allocation-free entry point: split-K partials in a static device array --------------------
//
// For callers that cannot allocate (code under graph capture that must not call hipMalloc, tight
// serving loops): the split-K partials of cdna3_attn_decode_noalloc live in this file-scope array,
// one copy per GPU, held until the process ends. Host code never passes `scratch` itself (its
// host-side name is not a device address); it passes the address hipGetSymbolAddress returns for
// the current device, looked up once per device. The partials are written before they are read,
// so nothing needs clearing between calls.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];

int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return CDNA4_ERR_INVALID_VALUE;
    void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        // Two threads may race here on first use; both obtain the same address.
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (p == nullptr) return CDNA4_ERR_INVALID_VALUE;
        g_scratch_addr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return 0;
}

}  // namespace

// Plan identity for replayed launches: two cache lengths with the same key launch the same grid
// with the same arguments apart from the length itself. -1 for an invalid configuration.
long long attn_decode_plan_key(const cdna3_decode_cfg& c) {
    Plan p;
    if (!plan_decode(c, true, p)) return -1;
    return p.wg ? (p.nt ? 3 : 1) : ((long long)p.P << 32) | (long long)p.KPW;
}

// The launches of cdna3_attn_decode planned for cfg->N, but with the cache length read on the
// device (*len_pos + 1) when they run, so that a captured graph of them serves every length with
// the same plan key. Used by the runtime's captured decode step; no validation beyond the plan.
int attn_decode_replayable(const void* q, const void* K, const void* V, void* o, const cdna3_decode_cfg& c, int dtype,
                           void* ws, size_t ws_bytes, const int* len_pos, hipStream_t s) {
    Plan p;
    if (!plan_decode(c, true, p) || !len_pos || ws_bytes < p.ws_bytes + 256) return CDNA4_ERR_INVALID_VALUE;
    const bool bf = dtype == CDNA4_BF16;
    if (c.D == 128) return bf ? launch_decode<128, true>(c, p, q, K, V, o, ws, s, len_pos)
                              : launch_decode<128, false>(c, p, q, K, V, o, ws, s, len_pos);
    return bf ? launch_decode<64, true>(c, p, q, K, V, o, ws, s, len_pos)
              : launch_decode<64, false>(c, p, q, K, V, o, ws, s, len_pos);
}

// Batch-1 decode attention left as P split-K partials for a consumer that merges them (the
// runtime's O-projection GEMV, llm_gemv_residual_merge): P workgroups per (kv head, head group),
// each over one of P key ranges of the cache (*len_pos + 1 keys when len_pos is set, else c.N),
// writing part_ml [nQH][P][2] and part_o [nQH][P][D] at the start of ws. A short cache then runs
// on P times the workgroups of the one-launch plan, with no merge launch of its own. Bytes of ws:
// attn_decode_partials_bytes.
size_t attn_decode_partials_bytes(const cdna3_decode_cfg& c, int P) {
    const size_t nml = (size_t)c.nQHeads * P * 2;
    return ((nml * sizeof(float) + 255) & ~(size_t)255) + (size_t)c.nQHeads * P * c.D * sizeof(float);
}

int attn_decode_partials(const void* q, const void* K, const void* V, const cdna3_decode_cfg& c, int dtype, int P,
                         void* ws, size_t ws_bytes, const int* len_pos, hipStream_t s) {
    Plan p;
    if (!plan_decode(c, false, p) || c.batch != 1 || P < 1 || P > 65535 || !ws) return CDNA4_ERR_INVALID_VALUE;
    if (ws_bytes < attn_decode_partials_bytes(c, P)) return CDNA4_ERR_INVALID_VALUE;
    DecodeArgs a;
    a.len_pos = len_pos;
    a.q = q; a.K = K; a.V = V;
    a.part_ml = (float*)ws;
    a.part_o = (float*)((char*)ws + (((size_t)c.nQHeads * P * 2 * sizeof(float) + 255) & ~(size_t)255));
    a.N = c.N; a.nQH = c.nQHeads; a.nKVH = c.nKVHeads; a.stride = c.stride_kv == 0 ? c.N : c.stride_kv;
    a.G = p.G; a.HB = p.HB; a.KPW = 0; a.P = P;
    a.sc = kLog2e / sqrtf((float)c.D);
    const long long gy = (long long)c.nKVHeads * p.HB;
    if (gy > 65535) return CDNA4_ERR_INVALID_VALUE;
    const dim3 grid((unsigned)P, (unsigned)gy, 1u);
    const bool bf = dtype == CDNA4_BF16;
    if (c.D == 128) {
        constexpr int W = wg_waves<128>();
        if (bf) decode_wg<128, true, W, false, true><<<grid, 64 * W, 0, s>>>(a, nullptr);
        else decode_wg<128, false, W, false, true><<<grid, 64 * W, 0, s>>>(a, nullptr);
    } else {
        constexpr int W = wg_waves<64>();
        if (bf) decode_wg<64, true, W, false, true><<<grid, 64 * W, 0, s>>>(a, nullptr);
        else decode_wg<64, false, W, false, true><<<grid, 64 * W, 0, s>>>(a, nullptr);
    }
    return launch_status();
}

}  // namespace cdna4

using namespace cdna4;

extern "C" size_t cdna3_attn_decode_workspace_size(const cdna3_decode_cfg* cfg) {
    Plan p;
    if (!cfg || !plan_decode(*cfg, true, p)) return 0;
    return p.ws_bytes + 256;
}

extern "C" int cdna3_attn_decode(const void* q, const void* K, const void* V, void* o, const cdna3_decode_cfg* cfg,
                                 int dtype, void* workspace, size_t ws_bytes, cdna4_stream_t stream) {
    Plan p;
    if (!cfg || !plan_decode(*cfg, workspace != nullptr, p)) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_decode_args(q, K, V, o, dtype)) return e;
    if (workspace != nullptr && ws_bytes < p.ws_bytes + 256) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    return run_decode(*cfg, p, q, K, V, o, dtype, workspace, (hipStream_t)stream);
}

extern "C" int cdna3_attn_decode_plan(const cdna3_decode_cfg* cfg, int dtype, int with_workspace,
                                      cdna3_plan_info* out) {
    Plan p;
    if (!cfg || !out || !plan_decode(*cfg, with_workspace != 0, p)) return CDNA4_ERR_INVALID_VALUE;
    if (dtype != CDNA4_F16 && dtype != CDNA4_BF16) return CDNA4_ERR_INVALID_VALUE;
    out->kernel = p.wg ? CDNA4_KERNEL_DECODE_WG : CDNA4_KERNEL_DECODE_SPLIT;
    out->waves = p.wg ? (cfg->D == 64 ? wg_waves<64>() : wg_waves<128>()) : 1;
    out->rows = p.KPW;
    out->partials = p.P;
    out->grid = (long long)p.P * cfg->nKVHeads * p.HB * cfg->batch;
    out->workspace = p.wg ? 0 : p.ws_bytes + 256;
    return 0;
}

extern "C" size_t cdna3_attn_decode_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int cdna3_attn_decode_noalloc(const void* q, const void* K, const void* V, void* o,
                                         const cdna3_decode_cfg* cfg, int dtype, cdna4_stream_t stream) {
    Plan p;
    if (!cfg || !plan_decode(*cfg, true, p)) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_decode_args(q, K, V, o, dtype)) return e;
    const size_t need = p.wg ? 0 : p.ws_bytes + 256;
    if (need > kScratchBytes) return CDNA4_ERR_SCRATCH_TOO_SMALL;
    if (int e = check_device()) return e;
    void* ws = nullptr;
    if (!p.wg) {
        if (int e = scratch_address(&ws)) return e;
    }
    return run_decode(*cfg, p, q, K, V, o, dtype, ws, (hipStream_t)stream);
}
