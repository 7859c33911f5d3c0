// MFMA attention tile machinery shared by the prefill and decode kernels (gfx950).
//
// Orientation: S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_{f16,bf16}. The S^T
// accumulator of a lane holds one query column (q = lane % 16) and 4 keys, so the softmax
// state of a query and its O^T accumulator live in the same lanes, and P goes from the S^T
// accumulator into the B operand of the P.V MFMA without data movement: the rows of each K
// operand tile are permuted (key = 8*(m/4) + 4*u + m%4 for A-row m of sub-tile u) so that the
// 8 keys a lane holds are the 8 consecutive keys its B operand needs. K rows come from LDS with
// ds_read_b128 under the swizzle swz_k<D>, V^T rows with ds_read_b64_tr_b16 under swz_v<D>,
// both free of bank conflicts.
// Softmax runs in base 2 (scores prescaled by log2(e) / sqrt(D)) against a lazily refreshed
// reference maximum m (see kTau).
#pragma once
#include "common.hpp"
#include "wave_primitives/detail/xlane.hpp"
#include <math.h>

namespace cdna4 {
namespace tile {

using wave::xlane::cross_row_allreduce;
using wave::xlane::Max;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#define LDS_AS __attribute__((address_space(3)))
typedef LDS_AS void LDS_AS_T;   // pointee type of an LDS address

constexpr float kLog2e = 1.4426950408889634f;


template <bool kBf16>
__device__ __forceinline__ f32x4 mfma(const u32x4& a, const u32x4& b, const f32x4& c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> one dword of two 16-bit values, round to nearest even
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    const f32x2 v = {a, b};
    if constexpr (kBf16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// XOR swizzles of the 16-byte chunks of key row r inside a K tile (swz_k) and a V tile (swz_v).
// The LDS has 64 four-byte banks (256 bytes per clock). Both swizzles depend on row bits 0, 1,
// 3 and 4 only (see LdsOffsets).
//   * K operand reads (ds_read_b128, 4 clocks per wave): lane (li, g) reads row
//     r = 8*(li/4) + li%4 (+ 4u + 32kc) at chunk g + 4c. Which 16 lanes share a clock is not
//     documented; measured on gfx950, a swizzle that spreads every 16 consecutive lanes over the
//     16 chunk positions still leaves a 2-way conflict (8 clocks per read), and one that is
//     conflict-free under every pairing of 8-lane blocks consistent with that measurement runs
//     at 4 clocks with no conflict cycles (SQ_LDS_BANK_CONFLICT = 0). That is swz_k:
//     D = 128 (16 chunks per 256-byte row): bits 0-1 <- r0-r1, bits 2-3 <- r3-r4;
//     D = 64 (8 chunks per 128-byte row, two rows per 256-byte window): bits 0-2 <- r1, r3, r4.
//   * V^T operand reads (ds_read_b64_tr_b16, 2 clocks): a lane group reads rows 8g + x
//     (x = 0..3) at two adjacent chunks; the 4 rows must land on distinct chunk pairs, and lane
//     groups g, g+1 (one 32-lane pass) on different 128-byte halves. swz_v:
//     D = 128: bit 0 <- r4, bits 1-2 <- r0-r1, bit 3 <- r3;
//     D = 64: bit 0 <- r4, bit 1 <- r1, bit 2 <- r3 (measured conflict-free as well).
template <int D>
__device__ __forceinline__ int swz_k(int r) {
    if constexpr (D == 128)
        return (r & 3) | (((r >> 3) & 3) << 2);
    else
        return ((r >> 1) & 1) | (((r >> 3) & 1) << 1) | (((r >> 4) & 1) << 2);
}
template <int D>
__device__ __forceinline__ int swz_v(int r) {
    if constexpr (D == 128)
        return ((r >> 4) & 1) | ((r & 3) << 1) | (((r >> 3) & 1) << 3);
    else
        return ((r >> 4) & 1) | (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}
// Swizzle of a tile that holds K rows (kIsK) or V rows.
template <int D, bool kIsK>
__device__ __forceinline__ int swz(int r) {
    return kIsK ? swz_k<D>(r) : swz_v<D>(r);
}

// Softmax reference maxima are refreshed only when a new maximum exceeds them by more than
// kTau (base-2 units): p = 2^(s - m) then stays <= 2^kTau, and O and l, accumulated against the
// same reference, give the exact O / l; most tiles skip the rescale of O entirely.
constexpr float kTau = 8.f;
// Initial reference maximum: finite, so no -inf - -inf can arise; the first chunk with a visible
// key always exceeds it by more than kTau and replaces it (alpha = 2^(kInitM - m) = 0), and masked
// scores (-inf) give p = 0 against it.
constexpr float kInitM = -1e30f;

// Per-lane byte offsets of the LDS operand reads within one K or V tile. The swizzle of a row
// depends only on bits 0, 1, 3, 4 of its index, which come from the lane alone, so the offsets of
// every sub-tile u, key chunk kc and (for V) row r + 4 differ from these by a compile-time
// constant (folded into the ds_read immediate). Within a row, d chunk c of the K operand sits at
// k ^ (c << 6) and d tile dt of the V^T operand at v ^ (dt << 5): the chunk index occupies offset
// bits that the row base and the swizzled low bits do not touch.
struct LdsOffsets {
    uint32_t k;   // K operand: d chunk 0, sub-tile 0, key chunk 0
    uint32_t v;   // first V^T transpose read: d tile 0, key chunk 0
    __device__ __forceinline__ uint32_t kc(int c) const { return k ^ ((uint32_t)c << 6); }
    __device__ __forceinline__ uint32_t vd(int dt) const { return v ^ ((uint32_t)dt << 5); }
};

template <int D>
__device__ __forceinline__ LdsOffsets lds_offsets(int li, int g) {
    LdsOffsets off;
    const int rk = (li >> 2) * 8 + (li & 3);                 // K row of A-row li, sub-tile 0
    off.k = (uint32_t)(rk * D + ((g ^ swz_k<D>(rk)) * 8)) * 2u;
    const int rv = g * 8 + (li >> 2);                        // V row of the first transpose read
    off.v = (uint32_t)(rv * D + ((((li & 3) >> 1) ^ swz_v<D>(rv)) * 8) + (li & 1) * 4) * 2u;
    return off;
}

// S^T = K Q^T for chunk kc of tile Kt: s[t][u][e] is key 32kc + 8g + 4u + e of the tile.
template <int D, int QT, bool kBf16>
__device__ __forceinline__ void qk_chunk(const char* Kt, const LdsOffsets& off, const u32x4 (&qb)[QT][D / 32],
                                         f32x4 (&s)[QT][2], int kc) {
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) s[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const u32x4 ka = *(const u32x4*)(Kt + off.kc(c) + (kc * 32 + u * 4) * D * 2);
#pragma unroll
            for (int t = 0; t < QT; ++t) s[t][u] = mfma<kBf16>(ka, qb[t][c], s[t][u]);
        }
}

// Masks a chunk whose first key is kb (diagonal / ragged chunks only) and returns, per lane, the
// raw maxima lm and whether some score exceeds its query's reference maximum by more than kTau.
template <int QT, bool kMask>
__device__ __forceinline__ bool check_chunk(f32x4 (&s)[QT][2], const float (&m)[QT], float (&lm)[QT], int kb,
                                            int qw0, int seqK, int causal, float sc, int li, int g) {
    bool need = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float v = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (kMask) {
                    const int key = kb + g * 8 + u * 4 + e;
                    const int q = qw0 + t * 16 + li;
                    if (key >= seqK || (causal && key > q)) s[t][u][e] = -INFINITY;
                }
                v = fmaxf(v, s[t][u][e]);
            }
        lm[t] = v;
        need |= v * sc > m[t] + kTau;
    }
    return need;
}

// New reference maxima (uniform over the four lanes of a query) and rescale of O and l.
template <int D, int QT>
__device__ __forceinline__ void rescale_rows(const float (&lm)[QT], float (&m)[QT], f32x4 (&o)[QT][D / 16],
                                             f32x4 (&lacc)[QT], float sc) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const float mx = cross_row_allreduce(lm[t], Max{}) * sc;
        const float mn = (mx > m[t] + kTau) ? mx : m[t];
        const float alpha = __builtin_amdgcn_exp2f(m[t] - mn);   // 0 while m is kInitM
        m[t] = mn;
        lacc[t] *= alpha;
#pragma unroll
        for (int d = 0; d < D / 16; ++d) o[t][d] *= alpha;
    }
}

// P = 2^(s sc - m) packed into the B operands of the P.V MFMA.
template <int QT, bool kBf16>
__device__ __forceinline__ void softmax_chunk(const f32x4 (&s)[QT][2], const float (&m)[QT], u32x4 (&pb)[QT],
                                              float sc) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float p[8];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) p[u * 4 + e] = __builtin_amdgcn_exp2f(fmaf(s[t][u][e], sc, -m[t]));
        pb[t] = u32x4{pack2<kBf16>(p[0], p[1]), pack2<kBf16>(p[2], p[3]), pack2<kBf16>(p[4], p[5]),
                      pack2<kBf16>(p[6], p[7])};
    }
}

// Keys below kLoKeys enter the bf16 P.V product with a second weight term. A weight rounded to
// bf16 carries 8 significant bits, and the output moves by up to 2^-9 sum_i w_i |v_i - O| (w_i
// the normalised weights): a query that sees only a few keys (the first rows of a causal
// sequence, a short cache) can be off by ~3e-3 for N(0,1) values. Sent as hi = bf16(p) plus
// lo = bf16(p - hi) (p - hi is exact in fp32), a weight carries ~16 bits, and the two-term chunk
// costs one more set of P.V and row-sum MFMAs. A query that sees more than kLoKeys keys spreads
// its weight so that the rounding of the later keys averages out (its error falls as one over the
// square root of the number of keys weighted alike), so only the first keys of a stream need it.
constexpr int kLoKeys = 64;

// The second term: lo = bf16(p - bf16(p)) for the weights softmax_chunk forms from the same s and
// m (bit-identical p), packed like its B operands. fp16 weights (11 bits) need no second term.
template <int QT>
__device__ __forceinline__ void softmax_lo_chunk(const f32x4 (&s)[QT][2], const float (&m)[QT], u32x4 (&pl)[QT],
                                                 float sc) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[t][x >> 1][(x & 1) * 2], sc, -m[t]));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[t][x >> 1][(x & 1) * 2 + 1], sc, -m[t]));
            const uint32_t hi = pack2<true>(p0, p1);
            const float h0 = __builtin_bit_cast(float, hi << 16), h1 = __builtin_bit_cast(float, hi & 0xFFFF0000u);
            pl[t][x] = pack2<true>(p0 - h0, p1 - h1);
        }
    }
}

// O^T += V^T P^T for chunk kc of tile Vt, and l += row sums of P (ones-operand MFMA).
template <int D, int QT, bool kBf16>
__device__ __forceinline__ void pv_chunk(const char* Vt, const LdsOffsets& off, const u32x4 (&pb)[QT],
                                         f32x4 (&o)[QT][D / 16], f32x4 (&lacc)[QT], int kc) {
    const uint32_t one2 = kBf16 ? 0x3F803F80u : 0x3C003C00u;   // two 16-bit 1.0
#pragma unroll
    for (int t = 0; t < QT; ++t) lacc[t] = mfma<kBf16>(u32x4{one2, one2, one2, one2}, pb[t], lacc[t]);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(Vt + off.vd(dt) + (kc * 32) * D * 2));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(Vt + off.vd(dt) + (kc * 32 + 4) * D * 2));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 va = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
        for (int t = 0; t < QT; ++t) o[t][dt] = mfma<kBf16>(va, pb[t], o[t][dt]);
    }
}

}  // namespace tile
}  // namespace cdna4
