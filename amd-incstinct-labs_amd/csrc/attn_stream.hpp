// Streaming K/V through a per-wave LDS ring for the gfx950 attention kernels: asynchronous
// 16-byte global->LDS copies issued as inline assembly and waited for explicitly, the swizzled
// stage layout the tile reads expect, and the per-wave loop that folds a key range into a
// running base-2 (m, l, O) for 16 query columns on the matrix cores.
#pragma once
#include "attn_tile.hpp"

namespace cdna4 {
namespace stream {

using tile::f32x4;

constexpr int kDecT = 32;       // keys per chunk / ring stage
constexpr int kDecStages = 2;   // ring depth: one chunk in flight while the wave computes one

// One asynchronous copy, 16 bytes per lane: lane i's bytes at gsrc land at LDS lds_dst + 16 i
// (lds_dst wave-uniform, in M0). Issued as inline assembly so that the compiler does not track
// it (it would otherwise wait for every copy before any LDS read); the kernel waits itself.
// The compiler's hazard recognizer does not look inside inline assembly, so the copies keep
// their own wait states: an SALU write of M0 needs 1 before an LDS DMA (`s_nop 0`; the compiler
// writes M0 for the "{m0}" operand with an SALU move).
// kNT sets the copy's non-temporal (streaming) cache policy, for data read exactly once (the
// decode's K/V): a plain 1 GiB read stream measured ~7.0 TB/s with it against ~6.3 TB/s without on
// the MI355X, and the config-4 decode 5.8 -> 6.6 TB/s. Data that other workgroups re-read from L2
// (the prefill's K/V tiles) keep the default policy: with it the prefill lost 9 %.
template <bool kNT = false>
__device__ __forceinline__ void dma16(const void* gsrc, const void* lds_dst) {
    const uint32_t base = (uint32_t)(uintptr_t)(const tile::LDS_AS_T*)lds_dst;
    if constexpr (kNT)
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(gsrc), "{m0}"(base) : "memory");
    else
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gsrc), "{m0}"(base) : "memory");
}

// The same copy from a wave-uniform base (SGPR pair) plus a 32-bit per-lane byte offset: no
// per-copy 64-bit address arithmetic in the vector ALU. A VALU write of an SGPR (v_readlane of a
// spilled SGPR, v_readfirstlane) needs 5 wait states before a vector memory instruction reads that
// SGPR, and the compiler does not know the copy reads it; so the base is first moved by the SALU
// (which waits for VALU-written SGPRs by itself) into a fresh pair that only the copy reads.
__device__ __forceinline__ void dma16_s(const void* sbase, uint32_t voff, const void* lds_dst) {
    const uint32_t base = (uint32_t)(uintptr_t)(const tile::LDS_AS_T*)lds_dst;
    const void* b;
    asm volatile("s_mov_b64 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0"
                 : "=&s"(b) : "v"(voff), "s"(sbase), "{m0}"(base) : "memory");
}

// Wait until at most Y of this wave's newest copy groups (kCopies copies each) are in flight.
template <int kCopies>
__device__ __forceinline__ void wait_copies_younger(int y) {
    switch (y) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kCopies) : "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(%0)" : : "n"(2 * kCopies) : "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(%0)" : : "n"(3 * kCopies) : "memory"); break;
    }
}

// Copy keys [k0, k0 + kDecT) of one head (row stride rs elements; rows past N re-read key N-1,
// they are masked) into a ring stage, 16-byte chunks of a row XOR-swizzled as the tile reads expect
// (the K swizzle when kIsK, else the V swizzle); kNT: non-temporal copies (see dma16).
template <int D, bool kIsK, bool kNT = false>
__device__ __forceinline__ void load_stage(const uint16_t* __restrict__ head, long long rs, int k0, int N,
                                           uint16_t* stage, int lane) {
    constexpr int CPR = D / 8;
    constexpr int NI = kDecT * CPR / 64;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int p = j * 64 + lane;
        const int r = p / CPR;
        const int lc = (p % CPR) ^ tile::swz<D, kIsK>(r);
        const int key = min(k0 + r, N - 1);
        dma16<kNT>(head + key * rs + lc * 8, stage + j * 64 * 8);
    }
}

// The per-wave loop of the split-K decode kernel as a function (decode_mfma keeps its own copy,
// whose code generation the long-cache tuning was measured on), for the kernels that split a key
// range over the waves of a workgroup.
// One wave streams keys [kbeg, kend) of one kv head through its NS-stage LDS ring and leaves the
// unnormalised (m, l, O) of its query heads in registers: lane (li, g) holds
// O^T[16 dt + 4 g + e][head li] in o[0][dt][e], the running base-2 max of head li in m[0] and its
// denominator in lacc[0][0]. An empty range leaves m = kInitM, l = 0, O = 0.
// Keys are rows of K and V (row stride rs elements, N rows); the 16 B-operand columns of qb are
// 16 query heads (decode) or 16 query rows qw0 .. qw0 + 15 (prefill; causal masks key > query).
// kNT: non-temporal copies, for keys no other workgroup reads (see dma16).
template <int D, bool kBf16, int NS, bool kNT = false>
__device__ __forceinline__ void stream_keys(const uint16_t* Kh, const uint16_t* Vh, long long rs, int N, int kbeg,
                                            int kend, int qw0, int causal, float sc, const u32x4 (&qb)[1][D / 32],
                                            f32x4 (&o)[1][D / 16], f32x4 (&lacc)[1], float (&m)[1], uint16_t* k_lds,
                                            uint16_t* v_lds, int lane) {
    constexpr int NDT = D / 16;
    constexpr int kStage = kDecT * D;                 // elements per K (or V) stage
    constexpr int kCopies = 2 * kDecT * (D / 8) / 64;  // copies per stage (K and V)
    const int li = lane & 15, g = lane >> 4;
    const int nch = (kend - kbeg + kDecT - 1) / kDecT;   // <= 0 for an empty range
    m[0] = tile::kInitM;
    lacc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[0][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const tile::LdsOffsets off = tile::lds_offsets<D>(li, g);

#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < nch) {
            load_stage<D, true, kNT>(Kh, rs, kbeg + i * kDecT, N, k_lds + i * kStage, lane);
            load_stage<D, false, kNT>(Vh, rs, kbeg + i * kDecT, N, v_lds + i * kStage, lane);
        }
    int st = 0;   // stage of chunk ch
    for (int ch = 0; ch < nch; ++ch) {
        const int ahead = ch + NS - 1;
        if (ahead < nch) {
            const int sa = (st == 0) ? NS - 1 : st - 1;   // stage of chunk ch - 1, already consumed
            load_stage<D, true, kNT>(Kh, rs, kbeg + ahead * kDecT, N, k_lds + sa * kStage, lane);
            load_stage<D, false, kNT>(Vh, rs, kbeg + ahead * kDecT, N, v_lds + sa * kStage, lane);
        }
        wait_copies_younger<kCopies>(min(NS - 1, nch - 1 - ch));
        const char* Kt = (const char*)(k_lds + st * kStage);
        const char* Vt = (const char*)(v_lds + st * kStage);
        const int kb = kbeg + ch * kDecT;
        f32x4 s[1][2];
        tile::qk_chunk<D, 1, kBf16>(Kt, off, qb, s, 0);
        float lm[1];
        const bool need = (kb + kDecT > kend || (causal && kb + kDecT - 1 > qw0))
            ? tile::check_chunk<1, true>(s, m, lm, kb, qw0, kend, causal, sc, li, g)
            : tile::check_chunk<1, false>(s, m, lm, kb, qw0, kend, causal, sc, li, g);
        if (__builtin_amdgcn_ballot_w64(need)) tile::rescale_rows<D, 1>(lm, m, o, lacc, sc);
        u32x4 pb[1];
        tile::softmax_chunk<1, kBf16>(s, m, pb, sc);
        tile::pv_chunk<D, 1, kBf16>(Vt, off, pb, o, lacc, 0);
        if constexpr (kBf16) {
            if (kb < tile::kLoKeys) {   // the first keys: the weights' second bf16 term
                tile::softmax_lo_chunk<1>(s, m, pb, sc);
                tile::pv_chunk<D, 1, true>(Vt, off, pb, o, lacc, 0);
            }
        }
        st = (st == NS - 1) ? 0 : st + 1;
    }
}

// Workgroup merge after W waves have each run stream_keys over their own key range: the waves
// leave their (m, l, O) in LDS (po over the K rings, pml over the V rings, after a barrier that
// ends every ring's use), then all W * 64 lanes merge pairs of adjacent outputs,
// o = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w, and store them as 16-bit pairs to
// out[h * D + d] for the nrows query heads (columns) h < nrows.
template <int D, bool kBf16, int W>
__device__ __forceinline__ void merge_waves(const f32x4 (&o)[1][D / 16], const f32x4 (&lacc)[1], const float (&m)[1],
                                            float* po, float* pml, int nrows, uint16_t* out, int wave, int lane) {
    constexpr int NDT = D / 16;
    const int li = lane & 15, g = lane >> 4;
    __syncthreads();   // every wave is done with its ring: reuse the LDS for the partials
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
        *(f32x4*)(po + ((size_t)wave * 16 + li) * D + dt * 16 + g * 4) = o[0][dt];
    if (g == 0) {
        pml[(wave * 16 + li) * 2] = m[0];
        pml[(wave * 16 + li) * 2 + 1] = lacc[0][0];
    }
    __syncthreads();
    for (int p = (int)threadIdx.x; p < nrows * (D / 2); p += 64 * W) {
        const int h = p / (D / 2), d = 2 * (p % (D / 2));
        float M = tile::kInitM;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, pml[(w * 16 + h) * 2]);
        float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float wt = exp2f(pml[(w * 16 + h) * 2] - M);
            L = fmaf(wt, pml[(w * 16 + h) * 2 + 1], L);
            const float2 v = *(const float2*)(po + ((size_t)w * 16 + h) * D + d);
            o0 = fmaf(wt, v.x, o0);
            o1 = fmaf(wt, v.y, o1);
        }
        const float inv = L > 0.f ? 1.f / L : 1.f;
        *(uint32_t*)(out + (size_t)h * D + d) = tile::pack2<kBf16>(o0 * inv, o1 * inv);
    }
}

// merge_waves for a workgroup that serves one of several key ranges of its heads: the merged
// (M, L, O) of the W waves, unnormalised (O and L relative to 2^M, M in base-2 units), goes to the
// split-K partial layout, part_ml[(row * P + split) * 2] = (M, L) and part_o[(row * P + split) * D
// + d] = O[d] for the nrows query heads (rows) of the group, row = qrow0 + h.
template <int D, int W>
__device__ __forceinline__ void merge_waves_part(const f32x4 (&o)[1][D / 16], const f32x4 (&lacc)[1],
                                                 const float (&m)[1], float* po, float* pml, int nrows,
                                                 float* part_ml, float* part_o, size_t qrow0, int P, int split,
                                                 int wave, int lane) {
    constexpr int NDT = D / 16;
    const int li = lane & 15, g = lane >> 4;
    __syncthreads();   // every wave is done with its ring: reuse the LDS for the partials
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
        *(f32x4*)(po + ((size_t)wave * 16 + li) * D + dt * 16 + g * 4) = o[0][dt];
    if (g == 0) {
        pml[(wave * 16 + li) * 2] = m[0];
        pml[(wave * 16 + li) * 2 + 1] = lacc[0][0];
    }
    __syncthreads();
    for (int p = (int)threadIdx.x; p < nrows * (D / 2); p += 64 * W) {
        const int h = p / (D / 2), d = 2 * (p % (D / 2));
        float M = tile::kInitM;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, pml[(w * 16 + h) * 2]);
        float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float wt = exp2f(pml[(w * 16 + h) * 2] - M);
            L = fmaf(wt, pml[(w * 16 + h) * 2 + 1], L);
            const float2 v = *(const float2*)(po + ((size_t)w * 16 + h) * D + d);
            o0 = fmaf(wt, v.x, o0);
            o1 = fmaf(wt, v.y, o1);
        }
        const size_t pidx = (qrow0 + h) * (size_t)P + split;
        *(float2*)(part_o + pidx * D + d) = make_float2(o0, o1);
        if (d == 0) *(float2*)(part_ml + pidx * 2) = make_float2(M, L);
    }
}

}  // namespace stream
}  // namespace cdna4
