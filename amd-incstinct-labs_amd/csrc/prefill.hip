// FlashAttention-2 prefill for gfx950 (MI355X).
//
// Reference behaviour restated (cdna3-prims/include/cdna3/detail/fa_prefill_kernel.hpp:
// 43-177, launched by cdna3-prims/include/cdna3/attention.hpp:86-109): O = softmax(Q K^T /
// sqrt(D)) V per (batch, query head), query head h reads kv head h / (nQH / nKVH), causal
// mask "key > query -> excluded", fp32 softmax and accumulation, O / l with an l > 0 guard.
//
// MI355X design of the f16 / bf16 kernels (fa_pipe for large problems, fa_mfma for mid-size):
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_{f16,bf16}. In that orientation
//     the S^T accumulator of a lane holds one query column (q = lane % 16) and 4 keys, so
//     the softmax state (m, l) and the O^T accumulator of a query live in the same lanes:
//     the running rescale is a per-lane multiply, and P goes from the S^T accumulator
//     straight into the B operand of the P.V MFMA without any data movement, because the
//     rows of each K operand tile are permuted (key = 8*(m/4) + 4*t + m%4 for A-row m of
//     sub-tile t) so that the 8 keys a lane holds are the 8 consecutive keys its B operand
//     needs.
//   * The row max over a query's keys spans the lane's own registers and the three other
//     lanes that hold the same query (lanes q, q+16, q+32, q+48): two permlane swaps, only
//     when some score exceeds the lazily kept reference maximum by more than kTau.
//   * K and V tiles go HBM -> LDS with global_load_lds_dwordx4 (asynchronous, no VGPRs),
//     a tile or two ahead of their use (fa_mfma: two buffers; fa_pipe: a ring of three). The
//     16-byte chunks of a key row are XOR-swizzled so the K operand reads (ds_read_b128) and
//     the V^T operand reads (ds_read_b64_tr_b16) are both free of bank conflicts.
//   * fa_pipe software-pipelines the key loop: the exponentials of one 32-key chunk are
//     interleaved with the S^T MFMAs of the next, so VALU and matrix-core work overlap.
//   * Q stays in VGPRs as B operands for the whole kernel; softmax is base-2 with a
//     log2(e)-prescaled scale; causal blocks are issued heaviest first, with all q blocks
//     of a (batch, head) on the same XCD so its K/V stay in that XCD's L2.
// The fp32 kernel (fa_f32) serves the fp32 arm of the reference configuration (fp32 in and
// out, accuracy 1e-4) on the fp32 matrix-core instruction (v_mfma_f32_16x16x4_f32).
#include <type_traits>

#include "attn_tile.hpp"
#include "attn_stream.hpp"

namespace cdna4 {
namespace {

using wave::xlane::allreduce;
using wave::xlane::cross_row_allreduce;
using wave::xlane::Max;
using wave::xlane::Sum;

using namespace tile;
constexpr int kBc = 64;       // keys per K/V tile

// (batch * head, q block) of a workgroup in a grid of exactly nbh * nqb workgroups. Workgroups are
// dispatched round-robin over the 8 XCDs (XCD = blockIdx % 8); with xcd_map (nbh % 8 == 0) the q
// blocks of (batch, head) bh all run on XCD bh % 8, so that head's K and V are fetched into one
// XCD's L2 instead of into all eight. Otherwise q blocks of one head are consecutive.
__device__ __forceinline__ void block_item(int item, int nqb, int xcd_map, int& bh, int& qblk) {
    if (xcd_map) {
        const int xcd = item & 7, slot = item >> 3;
        bh = (slot / nqb) * 8 + xcd;
        qblk = slot % nqb;
    } else {
        bh = item / nqb;
        qblk = item % nqb;
    }
}

struct PrefillArgs {
    const uint16_t* Q; const uint16_t* K; const uint16_t* V; uint16_t* O;
    // Element strides (batch, head, row) of Q, of K and V, and of O; the contiguous layout is
    // head = seq * D, batch = heads * seq * D, row = D.
    long long q_bs, q_hs, q_rs, k_bs, k_hs, k_rs, o_bs, o_hs, o_rs;
    int seqQ, seqK, nQH, nKVH, batch, causal;
    int nqb;          // q blocks per (batch, head)
    int xcd_map;      // 1: all q blocks of a (batch, head) on one XCD, heads in sequence
    int copy32;       // 1: a K/V tile's rows span < 4 GiB (32-bit per-lane copy offsets)
    float sc;         // log2(e) / sqrt(D)
};

// Issue the asynchronous copy of keys [k0, k0 + kBc) of one head into an LDS tile, chunks
// placed by the K (kIsK) or the V swizzle.
template <int D, int W, bool kIsK>
__device__ __forceinline__ void load_tile(const uint16_t* __restrict__ head, long long row_stride, int k0, int seqK,
                                          uint16_t* tile, int wave, int lane) {
    constexpr int CPR = D / 8;                       // 16-byte chunks per key row
    constexpr int NI = kBc * CPR / (64 * W);         // wave instructions per tile
    static_assert(NI >= 1 && NI * 64 * W == kBc * CPR, "tile copy must split evenly over the waves");
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int p0 = (j * W + wave) * 64;
        const int p = p0 + lane;
        const int r = p / CPR;
        const int lc = (p % CPR) ^ swz<D, kIsK>(r);
        const int key = min(k0 + r, seqK - 1);   // rows past the end re-read the last key (masked)
        __builtin_amdgcn_global_load_lds((const void*)(head + key * row_stride + lc * 8),
                                         (LDS_AS void*)(tile + p0 * 8), 16, 0, 0);
    }
}

// One 32-key half (kc) of a K/V tile: S^T MFMAs, masking, lazy rescale, P, P.V MFMAs.
template <int D, int QT, bool kBf16, bool kMask, bool kTwo = false>
__device__ __forceinline__ void chunk_body(const char* Kt, const char* Vt, const LdsOffsets& off,
                                           const u32x4 (&qb)[QT][D / 32],
                                           f32x4 (&o)[QT][D / 16], float (&m)[QT], f32x4 (&lacc)[QT], int kc,
                                           int k0, int qw0, int seqK, int causal, float sc, int li, int g) {
    constexpr int ND = D / 32;
    constexpr int NDT = D / 16;
    // ---- S^T = K Q^T: s[t][u][e] is key k0 + 32kc + 8g + 4u + e for query qw0 + 16t + li.
    f32x4 s[QT][2];
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) s[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < ND; ++c) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            // row kc*32 + 8*(li/4) + 4u + li%4, d chunk 4c + g (swizzled)
            const u32x4 ka = *(const u32x4*)(Kt + off.kc(c) + (kc * 32 + u * 4) * D * 2);
#pragma unroll
            for (int t = 0; t < QT; ++t) s[t][u] = mfma<kBf16>(ka, qb[t][c], s[t][u]);
        }
    }
    // ---- per-lane maxima of the raw scores (sc > 0 commutes with max), masked entries -> -inf.
    // Each lane checks its own scores against its query's reference maximum; only when some lane
    // of the wave sees one more than kTau above it does the wave form the cross-lane maxima
    // (uniform over the four lanes of a query) and rescale O and l.
    float lm[QT];
    bool need = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float v = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (kMask) {
                    const int key = k0 + kc * 32 + g * 8 + u * 4 + e;
                    const int q = qw0 + t * 16 + li;
                    if (key >= seqK || (causal && key > q)) s[t][u][e] = -INFINITY;
                }
                v = fmaxf(v, s[t][u][e]);
            }
        lm[t] = v;
        need |= v * sc > m[t] + kTau;
    }
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const float mx = cross_row_allreduce(lm[t], Max{}) * sc;
            const float mn = (mx > m[t] + kTau) ? mx : m[t];
            const float alpha = __builtin_amdgcn_exp2f(m[t] - mn);   // 0 while m is kInitM
            m[t] = mn;
            lacc[t] *= alpha;
#pragma unroll
            for (int d = 0; d < NDT; ++d) o[t][d] *= alpha;
        }
    }
    // ---- P = 2^(s sc - m), packed into the B operands of the P.V MFMA; l += row sums of exactly
    // the (rounded) weights the product uses, as an MFMA with an all-ones A operand: every lane
    // of a query's column receives the full sum over the chunk's 32 keys.
    u32x4 pb[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const float mref = m[t];
        float p[8];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) p[u * 4 + e] = __builtin_amdgcn_exp2f(fmaf(s[t][u][e], sc, -mref));
        pb[t] = u32x4{pack2<kBf16>(p[0], p[1]), pack2<kBf16>(p[2], p[3]), pack2<kBf16>(p[4], p[5]),
                      pack2<kBf16>(p[6], p[7])};
        const uint32_t one2 = kBf16 ? 0x3F803F80u : 0x3C003C00u;   // two 16-bit 1.0
        lacc[t] = mfma<kBf16>(u32x4{one2, one2, one2, one2}, pb[t], lacc[t]);
    }
    // ---- O^T += V^T P^T: A = V^T rows d, 8 consecutive keys per lane via transpose reads.
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        // rows r0 = kc*32 + 8g + li/4 and r0 + 4, d chunk 2dt + (li%4)/2 (swizzled), half li%2
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (LDS_AS s16x4*)(Vt + off.vd(dt) + (kc * 32) * D * 2));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (LDS_AS s16x4*)(Vt + off.vd(dt) + (kc * 32 + 4) * D * 2));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 va = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
        for (int t = 0; t < QT; ++t) o[t][dt] = mfma<kBf16>(va, pb[t], o[t][dt]);
    }
    // ---- kTwo (bf16, the tile of keys 0..63): the weights' second bf16 term, so that rows with
    // few keys keep fp32-level weights (see kLoKeys).
    if constexpr (kTwo) {
        softmax_lo_chunk<QT>(s, m, pb, sc);
        pv_chunk<D, QT, true>(Vt, off, pb, o, lacc, kc);
    }
}

template <int D, int QT, bool kBf16, bool kMask, bool kTwo = false>
__device__ __forceinline__ void tile_body(const char* Kt, const char* Vt, const LdsOffsets& off,
                                          const u32x4 (&qb)[QT][D / 32],
                                          f32x4 (&o)[QT][D / 16], float (&m)[QT], f32x4 (&lacc)[QT],
                                          int k0, int qw0, int seqK, int causal, float sc, int li, int g) {
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
        chunk_body<D, QT, kBf16, kMask, kTwo>(Kt, Vt, off, qb, o, m, lacc, kc, k0, qw0, seqK, causal, sc, li, g);
}

// One K/V tile: issue the asynchronous copy of the next tile into (kn, vn), then compute the
// current tile from (kt, vt). The four buffers are distinct, and saying so with __restrict__
// lets the compiler skip the wait for the copy before every read of the current tile.
template <int D, int W, int QT, bool kBf16>
__device__ __forceinline__ void tile_step(const uint16_t* __restrict__ kt, const uint16_t* __restrict__ vt,
                                          uint16_t* __restrict__ kn, uint16_t* __restrict__ vn, bool load_next,
                                          const uint16_t* Kh, const uint16_t* Vh, int k0, int wave_qmax,
                                          const PrefillArgs& a, const LdsOffsets& off, const u32x4 (&qb)[QT][D / 32],
                                          f32x4 (&o)[QT][D / 16], float (&m)[QT], f32x4 (&lacc)[QT], int qw0,
                                          int wave, int lane, int li, int g) {
    if (load_next) {
        load_tile<D, W, true>(Kh, a.k_rs, k0 + kBc, a.seqK, kn, wave, lane);
        load_tile<D, W, false>(Vh, a.k_rs, k0 + kBc, a.seqK, vn, wave, lane);
    }
    if (!(a.causal && k0 > wave_qmax)) {
        const bool need_mask = (a.causal && k0 + kBc - 1 > qw0) || (k0 + kBc > a.seqK);
        if (kBf16 && k0 < kLoKeys)   // keys 0..63 (kBc = 64): weights with a second bf16 term
            tile_body<D, QT, kBf16, true, kBf16>((const char*)kt, (const char*)vt, off, qb, o, m, lacc, k0, qw0, a.seqK, a.causal, a.sc, li, g);
        else if (need_mask)
            tile_body<D, QT, kBf16, true>((const char*)kt, (const char*)vt, off, qb, o, m, lacc, k0, qw0, a.seqK, a.causal, a.sc, li, g);
        else
            tile_body<D, QT, kBf16, false>((const char*)kt, (const char*)vt, off, qb, o, m, lacc, k0, qw0, a.seqK, a.causal, a.sc, li, g);
    }
}

template <int D, int W, int QT, bool kBf16>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void fa_mfma(PrefillArgs a) {
    constexpr int ND = D / 32;    // 32-wide d chunks (K dimension of S^T)
    constexpr int NDT = D / 16;   // 16-wide d tiles (M dimension of O^T)
    constexpr int BM = W * QT * 16;
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kBc * D];   // [buffer][K|V]

    const int lane = (int)(threadIdx.x & 63u);
    const int wave = (int)(threadIdx.x >> 6);
    const int li = lane & 15, g = lane >> 4;

    // Persistent grid: workgroup i takes work items i, i + gridDim.x, ... Item -> (batch, head,
    // q block): workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8) and the grid
    // is a multiple of 8, so item % 8 is the workgroup's XCD. With xcd_map, XCD x owns heads
    // x, x + 8, ... and its workgroups walk one head at a time, so they share that head's K/V in
    // the XCD's L2; within a head the q blocks go heaviest (causal) first, and the order flips
    // for every other head so that each workgroup's total work evens out.
    const int nbh = a.batch * a.nQH;
    const int nitems = nbh * a.nqb;
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
        int bh, qrev;
        if (a.xcd_map) {
            const int xcd = item & 7, slot = item >> 3;
            bh = (slot / a.nqb) * 8 + xcd;
            qrev = slot % a.nqb;
            if ((slot / a.nqb) & 1) qrev = a.nqb - 1 - qrev;
        } else {
            bh = item % nbh;
            qrev = item / nbh;
        }
        const int qblk = a.causal ? (a.nqb - 1 - qrev) : qrev;
        const int b = bh / a.nQH, h = bh % a.nQH;
        const int kvh = h / (a.nQH / a.nKVH);
        const int q0 = qblk * BM;
        const int qw0 = q0 + wave * QT * 16;   // first query row of this wave

        const uint16_t* Kh = a.K + b * a.k_bs + kvh * a.k_hs;
        const uint16_t* Vh = a.V + b * a.k_bs + kvh * a.k_hs;
        const uint16_t* Qh = a.Q + b * a.q_bs + h * a.q_hs;

        // Q as B operands: lane holds Q[q = qw0 + t*16 + li][32*c + 8*g .. +8].
        u32x4 qb[QT][ND];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const int q = min(qw0 + t * 16 + li, a.seqQ - 1);
#pragma unroll
            for (int c = 0; c < ND; ++c) {
                qb[t][c] = *(const u32x4*)(Qh + q * a.q_rs + c * 32 + g * 8);
            }
        }

        f32x4 o[QT][NDT], lacc[QT];
        float m[QT];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            m[t] = kInitM;
            lacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < NDT; ++d) {
                o[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }

        const LdsOffsets off = lds_offsets<D>(li, g);
        int ntiles = (a.seqK + kBc - 1) / kBc;
        if (a.causal) ntiles = min(ntiles, (min(q0 + BM, a.seqQ) - 1) / kBc + 1);
        const int wave_qmax = min(qw0 + QT * 16, a.seqQ) - 1;   // last real query of this wave

        load_tile<D, W, true>(Kh, a.k_rs, 0, a.seqK, lds[0][0], wave, lane);
        load_tile<D, W, false>(Vh, a.k_rs, 0, a.seqK, lds[0][1], wave, lane);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        for (int it = 0; it < ntiles; ++it) {
            const int buf = it & 1;
            tile_step<D, W, QT, kBf16>(lds[buf][0], lds[buf][1], lds[buf ^ 1][0], lds[buf ^ 1][1], it + 1 < ntiles, Kh, Vh,
                                       it * kBc, wave_qmax, a, off, qb, o, m, lacc, qw0, wave, lane, li, g);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }

        // ---- O = O^T / l: lane holds d = 16dt + 4g + e of query li, and its query's full l.
        uint16_t* Oh = a.O + b * a.o_bs + h * a.o_hs;
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const float lt = lacc[t][0];
            const float inv = (lt > 0.f) ? 1.f / lt : 1.f;
            const int q = qw0 + t * 16 + li;
            if (q < a.seqQ) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 w = u32x2{pack2<kBf16>(o[t][dt][0] * inv, o[t][dt][1] * inv),
                                          pack2<kBf16>(o[t][dt][2] * inv, o[t][dt][3] * inv)};
                    *(u32x2*)(Oh + q * a.o_rs + dt * 16 + g * 4) = w;
                }
            }
        }
        __syncthreads();   // every wave is done with the LDS buffers before the next item's first copy
    }
}

// ---- the 8-wave kernel: software-pipelined key loop (fa_pipe) -------------------------------
// A wave walks its keys in 32-key chunks. Region j of the loop does, in one straight block:
//   P_j = 2^(S_j sc - m) from s (S^T of chunk j, already masked and max-checked), packed into
//   the P.V B operands, with the exponentials placed between the S^T MFMAs of chunk j + 1 (its
//   K operand reads two ahead), so that the VALU work issues under matrix-core work instead of
//   after it; then l += rowsum(P_j) and O^T += V^T P_j^T (V^T operand reads two ahead); then the
//   max check of chunk j + 1 and, rarely, the rescale of O and l.
// K/V tiles (64 keys) stream HBM -> LDS in a ring of three buffers, one workgroup barrier per
// tile: region 2t reads tile t (S of chunk 2t + 1, P.V of chunk 2t); the barrier before region
// 2t + 1 makes tile t + 1 visible and frees tile t - 1's buffer (last read by region 2t - 1),
// which then receives the copy of tile t + 2; region 2t + 1 reads tiles t + 1 (S of chunk 2t + 2)
// and t (P.V of chunk 2t + 1). The copies are inline assembly, so the compiler neither tracks nor
// waits for them; the kernel waits with vmcnt before each barrier.
// Tiles whose regions need no mask for any wave of the workgroup (keys below its first query,
// and a full chunk ahead) run in a main loop unrolled over the three buffers (LDS offsets become
// immediates); the remaining diagonal / ragged tiles run in a tail loop that masks every chunk
// and lets each wave skip the chunks past its last query. Keeping the two loops apart keeps each
// region one block: variants joined inside the loop made the register allocator copy the O
// accumulators at every join.
constexpr int kPipeBufs = 3;

// Masks chunk scores s whose first key is kb: key >= seqK or (causal) key > query -> -inf.
template <int QT>
__device__ __forceinline__ void mask_chunk(f32x4 (&s)[QT][2], int kb, int qw0, int seqK, int causal, int li, int g) {
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = kb + g * 8 + u * 4 + e;
                const int q = qw0 + t * 16 + li;
                if (key >= seqK || (causal && key > q)) s[t][u][e] = -INFINITY;
            }
}

// Causal mask of the chunk whose first key is the wave's first query (kb == qw0, both multiples of
// 32): key - query = 4u + e - (16t + li - 8g) for lane (li, g), so the pattern is the same for every
// such chunk, 2 VALU per score instead of mask_chunk's general form. Chunks below qw0 need no
// causal mask, and those above it lie past the wave's last query (never used).
template <int QT>
__device__ __forceinline__ void mask_diag(f32x4 (&s)[QT][2], int li, int g) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const int dq = 16 * t + li - 8 * g;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (4 * u + e > dq) s[t][u][e] = -INFINITY;
    }
}

// Per-lane raw maxima lm of a chunk and whether one exceeds its query's threshold thr = (m + kTau)
// / sc, i.e. whether a scaled score exceeds the reference maximum by more than kTau (the
// threshold is kept in raw score units so that the check per chunk needs no multiply).
template <int QT>
__device__ __forceinline__ bool check_raw(const f32x4 (&s)[QT][2], const float (&thr)[QT], float (&lm)[QT]) {
    bool need = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float v = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) v = fmaxf(v, s[t][u][e]);
        lm[t] = v;
        need |= v > thr[t];
    }
    return need;
}

// rescale_rows, then the thresholds of the new reference maxima.
template <int D, int QT>
__device__ __forceinline__ void rescale_pipe(const float (&lm)[QT], float (&m)[QT], float (&thr)[QT],
                                             f32x4 (&o)[QT][D / 16], f32x4 (&lacc)[QT], float sc, float inv_sc) {
    rescale_rows<D, QT>(lm, m, o, lacc, sc);
#pragma unroll
    for (int t = 0; t < QT; ++t) thr[t] = (m[t] + kTau) * inv_sc;
}

// The copy of one full K/V tile a region issues between its MFMAs (kCopy): global bases of the
// tile's K and V rows, their LDS buffers, and the per-lane offsets of copy_offsets.
template <int NI>
struct TileCopy {
    const uint16_t* kg; const uint16_t* vg;
    uint16_t* kd; uint16_t* vd;
    const uint32_t* koff; const uint32_t* voff;
    int wave, W;
    __device__ __forceinline__ void issue(int c) const {   // copy c of 2 NI: K parts, then V parts
        const int j = c % NI;
        if (c < NI) stream::dma16_s(kg, koff[j], kd + (j * W + wave) * 64 * 8);
        else stream::dma16_s(vg, voff[j], vd + (j * W + wave) * 64 * 8);
    }
};

// Region j (see above). Kn (K tile of chunk j + 1, half kcn) always points into the LDS ring;
// when chunk j + 1 does not exist for this wave (has_next false, tail only) the scores formed
// from it are ignored. Vc / kcc: V tile and half of chunk j. kTail: mask chunk j + 1. kTwo (bf16,
// tail tile 0 only): chunk j also enters with its weights' second bf16 term (see kLoKeys).
template <int D, int QT, bool kBf16, bool kTail, bool kCopy, int NI, bool kTwo = false>
__device__ __forceinline__ void pipe_region(const char* Kn, int kcn, const char* Vc, int kcc, const LdsOffsets& off,
                                           const u32x4 (&qb)[QT][D / 32], f32x4 (&s)[QT][2], f32x4 (&o)[QT][D / 16],
                                           float (&m)[QT], float (&thr)[QT], f32x4 (&lacc)[QT], const u32x4& ones,
                                           bool has_next, int kbn, int qw0, int seqK, int causal, float sc,
                                           float inv_sc, int li, int g, const TileCopy<NI>& cp) {
    constexpr int NK = (D / 32) * 2;   // K operand reads (ds_read_b128) of chunk j + 1, i = 2c + u
    constexpr int NV = D / 16;         // V^T operands of chunk j (two transpose reads each)
    constexpr int NP = QT * 8;         // P_j values per lane
    constexpr int SL = NP / NK;        // P values per interleave slot
    constexpr int kAhead = 2;          // LDS operand reads issued ahead of their MFMAs
    static_assert(NP % NK == 0 && SL % 2 == 0, "softmax slices must pair up for the packing");
    if constexpr (kTwo) {
        // Chunk j's keys lie below kLoKeys: first the P.V product of its weights' second bf16 term
        // (s holds chunk j's masked scores, m is the reference P_j is formed against; the sum into
        // O and l does not depend on the order), before chunk j + 1's scores are live.
        u32x4 pl[QT];
        softmax_lo_chunk<QT>(s, m, pl, sc);
        pv_chunk<D, QT, true>(Vc, off, pl, o, lacc, kcc);
        __builtin_amdgcn_sched_barrier(0);   // the region's reads stay after this block
    }
    float p[QT][8];
    u32x4 pb[QT];
    f32x4 sn[QT][2];
    u32x4 ka[NK];
    auto kread = [&](int i) {
        ka[i] = *(const u32x4*)(Kn + off.kc(i >> 1) + (kcn * 32 + (i & 1) * 4) * D * 2);
    };
    auto soft = [&](int v) {   // P value v (query tile v / 8, element v % 8)
        const int t = v >> 3, x = v & 7;
        p[t][x] = __builtin_amdgcn_exp2f(fmaf(s[t][x >> 2][x & 3], sc, -m[t]));
        if (x & 1) pb[t][x >> 1] = pack2<kBf16>(p[t][x - 1], p[t][x]);
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) kread(i);
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) sn[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    // S^T of chunk j + 1, one K operand (QT MFMAs) per slot, SL values of P_j per slot. The
    // scheduling barriers keep the slots in this order.
    // Wave priority 2 here, 1 for the P.V part, 0 for the check and the copies between regions:
    // measured +1.7 to +2.7 % on the causal B4 H32 S8192 D128 prefill over equal priorities.
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < QT; ++t) sn[t][i & 1] = mfma<kBf16>(ka[i], qb[t][i >> 1], sn[t][i & 1]);
        if (i + kAhead < NK) kread(i + kAhead);
        // one copy of the next-but-one tile per odd slot (NK / 2 = 2 NI slots): the waves' copies
        // then reach the texture unit spread over the region instead of all after the barrier
        if constexpr (kCopy) {
            static_assert(NK / 2 == 2 * NI, "one copy per odd slot");
            if (i & 1) cp.issue(i >> 1);
        }
#pragma unroll
        for (int v = 0; v < SL; ++v) soft(i * SL + v);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 va[NV];
    auto vread = [&](int dt) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(Vc + off.vd(dt) + (kcc * 32) * D * 2));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(Vc + off.vd(dt) + (kcc * 32 + 4) * D * 2));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        va[dt] = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
    };
#pragma unroll
    for (int dt = 0; dt < kAhead; ++dt) vread(dt);
    __builtin_amdgcn_s_setprio(1);
    // l += row sums of exactly the rounded weights the product uses (all-ones A operand)
#pragma unroll
    for (int t = 0; t < QT; ++t) lacc[t] = mfma<kBf16>(ones, pb[t], lacc[t]);
#pragma unroll
    for (int dt = 0; dt < NV; ++dt) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < QT; ++t) o[t][dt] = mfma<kBf16>(va[dt], pb[t], o[t][dt]);
        if (dt + kAhead < NV) vread(dt + kAhead);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    if constexpr (kTail) {   // wave-uniform branches: most tail chunks need neither mask
        if (causal && kbn == qw0) mask_diag<QT>(sn, li, g);
        if (kbn + 32 > seqK) mask_chunk<QT>(sn, kbn, qw0, seqK, causal, li, g);
    }
    float lm[QT];
    bool need = check_raw<QT>(sn, thr, lm);
    if constexpr (kTail) need = need && has_next;
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) s[t][u] = sn[t][u];
    if (__builtin_amdgcn_ballot_w64(need)) rescale_pipe<D, QT>(lm, m, thr, o, lacc, sc, inv_sc);
}

// Asynchronous copy of keys [k0, k0 + kBc) of one head into an LDS tile (inline assembly, see
// stream::dma16), chunks placed by the K (kIsK) or the V swizzle.
template <int D, int W, bool kIsK>
__device__ __forceinline__ void copy_tile(const uint16_t* __restrict__ head, long long row_stride, int k0, int seqK,
                                          uint16_t* tile, int wave, int lane) {
    constexpr int CPR = D / 8;
    constexpr int NI = kBc * CPR / (64 * W);
    static_assert(NI >= 1 && NI * 64 * W == kBc * CPR, "tile copy must split evenly over the waves");
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int p0 = (j * W + wave) * 64;
        const int p = p0 + lane;
        const int r = p / CPR;
        const int lc = (p % CPR) ^ swz<D, kIsK>(r);
        const int key = min(k0 + r, seqK - 1);   // rows past the end re-read the last key (masked)
        stream::dma16(head + key * row_stride + lc * 8, tile + p0 * 8);
    }
}

// Per-lane byte offsets of the copy of a full tile (row r, swizzled 16-byte chunk lc), the same for
// every tile of a head, so formed once per work item: a full tile's copies then need only a
// wave-uniform base (stream::dma16_s).
template <int D, int W, bool kIsK>
__device__ __forceinline__ void copy_offsets(long long row_stride, int wave, int lane,
                                             uint32_t (&voff)[kBc * (D / 8) / (64 * W)]) {
    constexpr int CPR = D / 8;
    constexpr int NI = kBc * CPR / (64 * W);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int p = (j * W + wave) * 64 + lane;
        const int r = p / CPR;
        const int lc = (p % CPR) ^ swz<D, kIsK>(r);
        voff[j] = (uint32_t)(((long long)r * row_stride + lc * 8) * 2);
    }
}

// Copy of keys [k0, k0 + kBc), all inside the sequence, with the offsets above.
template <int D, int W>
__device__ __forceinline__ void copy_tile_full(const uint16_t* head, long long row_stride, int k0,
                                               const uint32_t (&voff)[kBc * (D / 8) / (64 * W)], uint16_t* tile,
                                               int wave) {
    constexpr int NI = kBc * (D / 8) / (64 * W);
    const uint16_t* base = head + (long long)k0 * row_stride;
#pragma unroll
    for (int j = 0; j < NI; ++j) stream::dma16_s(base, voff[j], tile + (j * W + wave) * 64 * 8);
}

// Work item of a persistent workgroup: item = round * gridDim.x + position. With xcd_map (grid
// and batch * heads multiples of 8) the XCD of position p is p % 8 and it owns heads x, x + 8, ...;
// the G = grid / 8 workgroups of an XCD take, in round r, G consecutive entries of that XCD's
// head-major, heaviest-first item list (so they share one or a few heads' K/V in the XCD's L2),
// and take them in reverse order on odd rounds, so that a workgroup that drew a heavy causal q
// block in one round draws a light one in the next whatever the ratio of q blocks per head to G.
// Without xcd_map: heads vary fastest, q blocks heaviest first.
__device__ __forceinline__ void persistent_item(int item, int nqb, int nbh, int xcd_map, int& bh, int& qrev) {
    if (xcd_map) {
        const int grid = (int)gridDim.x;
        const int r = item / grid, p = item - r * grid;
        const int xcd = p & 7, sp = p >> 3, G = grid >> 3;
        const int K = min(G, ((nbh * nqb) >> 3) - r * G);   // this round's entries per XCD
        const int idx = r * G + ((r & 1) ? K - 1 - sp : sp);
        bh = (idx / nqb) * 8 + xcd;
        qrev = idx % nqb;
    } else {
        bh = item % nbh;
        qrev = item / nbh;
    }
}

template <int D, int W, int QT, bool kBf16>
__global__ __launch_bounds__(64 * W) void fa_pipe(PrefillArgs a) {
    constexpr int ND = D / 32;
    constexpr int NDT = D / 16;
    constexpr int BM = W * QT * 16;
    constexpr int NB = kPipeBufs;
    constexpr int kTile = kBc * D;                              // elements of one K (or V) tile
    constexpr int kCopies = 2 * (kBc * (D / 8) / (64 * W));     // copy instructions per tile per wave
    __shared__ __attribute__((aligned(16))) uint16_t lds[NB * 2 * kTile];   // [buffer][K|V][tile]

    const int lane = (int)(threadIdx.x & 63u);
    // wave-uniform as far as the compiler knows too, so that branches on it stay scalar
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int li = lane & 15, g = lane >> 4;

    const int nbh = a.batch * a.nQH;
    const int nitems = nbh * a.nqb;
    // Query block of this wave: waves w and w + W/2 share a SIMD, so the second half takes the
    // blocks in reverse (on the causal diagonal each SIMD holds one early and one late block).
    const int wblk = wave < W / 2 ? wave : W + W / 2 - 1 - wave;
    struct Item { int b, h, q0, qw0; };
    auto item_of = [&](int item) {
        int bh, qrev;
        persistent_item(item, a.nqb, nbh, a.xcd_map, bh, qrev);
        const int qblk = a.causal ? (a.nqb - 1 - qrev) : qrev;
        Item it;
        it.b = bh / a.nQH;
        it.h = bh % a.nQH;
        it.q0 = qblk * BM;
        it.qw0 = it.q0 + wblk * QT * 16;   // first query row of this wave
        return it;
    };
    // Q as B operands: lane holds Q[q = qw0 + t*16 + li][32*c + 8*g .. +8]. An item's Q is loaded
    // at the end of the previous item (into the registers its Q no longer needs), so the loads are
    // in flight during that item's output stores and final barrier.
    u32x4 qb[QT][ND];
    auto load_q = [&](const Item& it) {
        const uint16_t* Qh = a.Q + it.b * a.q_bs + it.h * a.q_hs;
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const int q = min(it.qw0 + t * 16 + li, a.seqQ - 1);
#pragma unroll
            for (int c = 0; c < ND; ++c) qb[t][c] = *(const u32x4*)(Qh + q * a.q_rs + c * 32 + g * 8);
        }
    };
    // per-lane offsets of full-tile copies: the same for every item
    constexpr int NI = kBc * (D / 8) / (64 * W);
    uint32_t koff[NI], voff[NI];
    copy_offsets<D, W, true>(a.k_rs, wave, lane, koff);
    copy_offsets<D, W, false>(a.k_rs, wave, lane, voff);
    if ((int)blockIdx.x < nitems) load_q(item_of(blockIdx.x));
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
        const Item it = item_of(item);
        const int b = it.b, h = it.h, q0 = it.q0, qw0 = it.qw0;
        const int kvh = h / (a.nQH / a.nKVH);
        const uint16_t* Kh = a.K + b * a.k_bs + kvh * a.k_hs;
        const uint16_t* Vh = a.V + b * a.k_bs + kvh * a.k_hs;
        f32x4 o[QT][NDT], lacc[QT];
        float m[QT], thr[QT];
        const float inv_sc = 1.f / a.sc;
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            m[t] = kInitM;
            thr[t] = (kInitM + kTau) * inv_sc;
            lacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < NDT; ++d) o[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        int ntiles = (a.seqK + kBc - 1) / kBc;
        if (a.causal) ntiles = min(ntiles, (min(q0 + BM, a.seqQ) - 1) / kBc + 1);
        // Main tiles t < t_main: for every wave, chunks 2t + 1 and 2t + 2 (whose scores tile t's
        // regions form) lie below the workgroup's first query and a full chunk inside seqK.
        int t_main = a.seqK >= 96 ? (a.seqK - 96) / 64 + 1 : 0;
        if (a.causal) t_main = min(t_main, q0 >= 95 ? (q0 - 95) / 64 + 1 : 0);
        t_main = min(t_main, ntiles);
        // the main loop's second regions copy tile t + 2 between their MFMAs, so it runs only while
        // that tile exists and is full (and the 32-bit lane offsets apply)
        t_main = a.copy32 ? min(t_main, min(ntiles - 2, a.seqK / kBc - 2)) : 0;
        t_main = max(t_main, 0);
        const int wave_qmax = min(qw0 + QT * 16, a.seqQ) - 1;   // last real query of this wave
        const int kend = a.causal ? min(a.seqK, wave_qmax + 1) : a.seqK;
        const int nch = (kend + 31) / 32;                        // this wave's chunks (>= 1)

        auto copy = [&](int tt, int buf) {   // K and V of tile tt into LDS buffer buf
            uint16_t* kd = lds + buf * 2 * kTile;
            if (a.copy32 && (tt + 1) * kBc <= a.seqK) {
                copy_tile_full<D, W>(Kh, a.k_rs, tt * kBc, koff, kd, wave);
                copy_tile_full<D, W>(Vh, a.k_rs, tt * kBc, voff, kd + kTile, wave);
            } else {
                copy_tile<D, W, true>(Kh, a.k_rs, tt * kBc, a.seqK, kd, wave, lane);
                copy_tile<D, W, false>(Vh, a.k_rs, tt * kBc, a.seqK, kd + kTile, wave, lane);
            }
        };
        // tiles 0 .. NB - 2 in flight; issued after the Q loads, so vmcnt counts them last
#pragma unroll
        for (int i = 0; i < NB - 1; ++i)
            if (i < ntiles) copy(i, i);
        if (ntiles > 1) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kCopies) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();
        const LdsOffsets off = lds_offsets<D>(li, g);

        // S^T of chunk 0, its mask and max check (the first check always sets m)
        f32x4 s[QT][2];
        qk_chunk<D, QT, kBf16>((const char*)lds, off, qb, s, 0);
        {
            float lm[QT];
            if (32 > a.seqK || (a.causal && 31 > qw0)) mask_chunk<QT>(s, 0, qw0, a.seqK, a.causal, li, g);
            if (__builtin_amdgcn_ballot_w64(check_raw<QT>(s, thr, lm)))
                rescale_pipe<D, QT>(lm, m, thr, o, lacc, a.sc, inv_sc);
        }
        // the all-ones A operand of the row-sum MFMA, held in registers for the whole item
        u32x4 ones;
        {
            const uint32_t one2 = kBf16 ? 0x3F803F80u : 0x3C003C00u;
            ones = u32x4{one2, one2, one2, one2};
            asm volatile("" : "+v"(ones));
        }

        // tile t sits in buffer bc = t % NB (a literal in the unrolled main loop)
        auto tile_iter = [&](int t, auto tail, auto two, int bc) {
            constexpr bool kTail = decltype(tail)::value;
            constexpr bool kTwo = decltype(two)::value;
            const int bn = bc == NB - 1 ? 0 : bc + 1;   // buffer of tile t + 1
            const char* Kt = (const char*)(lds + bc * 2 * kTile);
            const char* Vt = (const char*)(lds + bc * 2 * kTile + kTile);
            const char* Kn = (const char*)(lds + bn * 2 * kTile);
            // region 2t: P of chunk 2t, S of chunk 2t + 1 (this tile, keys 32..63), P.V of chunk 2t
            const int j0 = 2 * t;
            const int bf = bc == 0 ? NB - 1 : bc - 1;   // tile t - 1's buffer, refilled with tile t + 2
            TileCopy<NI> cp{Kh + (long long)(t + 2) * kBc * a.k_rs, Vh + (long long)(t + 2) * kBc * a.k_rs,
                            lds + bf * 2 * kTile, lds + bf * 2 * kTile + kTile, koff, voff, wave, W};
            if (!kTail)
                pipe_region<D, QT, kBf16, false, false, NI>(Kt, 1, Vt, 0, off, qb, s, o, m, thr, lacc, ones, true,
                                                            (j0 + 1) * 32, qw0, a.seqK, a.causal, a.sc, inv_sc, li, g, cp);
            else if (j0 < nch)
                pipe_region<D, QT, kBf16, true, false, NI, kTwo>(Kt, 1, Vt, 0, off, qb, s, o, m, thr, lacc, ones, j0 + 1 < nch,
                                                           (j0 + 1) * 32, qw0, a.seqK, a.causal, a.sc, inv_sc, li, g, cp);
            if (!kTail || t + 1 < ntiles) {
                // tile t + 1 landed and is visible; every wave is past region 2t - 1, the last reader
                // of tile t - 1's buffer, which now receives tile t + 2 (in the tail here, in the main
                // loop during region 2t + 1)
                asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
                __syncthreads();
                if (kTail && t + 2 < ntiles) copy(t + 2, bf);
            }
            // region 2t + 1: P of chunk 2t + 1, S of chunk 2t + 2 (tile t + 1, keys 0..31), P.V of
            // chunk 2t + 1; past the last tile Kn is a stale buffer whose scores are ignored
            const int j1 = 2 * t + 1;
            if (!kTail)
                pipe_region<D, QT, kBf16, false, true, NI>(Kn, 0, Vt, 1, off, qb, s, o, m, thr, lacc, ones, true,
                                                           (j1 + 1) * 32, qw0, a.seqK, a.causal, a.sc, inv_sc, li, g, cp);
            else if (j1 < nch)
                pipe_region<D, QT, kBf16, true, false, NI, kTwo>(Kn, 0, Vt, 1, off, qb, s, o, m, thr, lacc, ones, j1 + 1 < nch,
                                                           (j1 + 1) * 32, qw0, a.seqK, a.causal, a.sc, inv_sc, li, g, cp);
        };
        int t = 0;
        for (; t + NB <= t_main; t += NB) {
#pragma unroll
            for (int i = 0; i < NB; ++i) tile_iter(t + i, std::false_type{}, std::false_type{}, i);
        }
        for (; t < t_main; ++t) tile_iter(t, std::false_type{}, std::false_type{}, t % NB);
        // bf16: keys 0..63 (tile 0, reached in the tail only when the main loop is empty) enter
        // with their weights' second bf16 term, in a copy of the tail step of its own
        if constexpr (kBf16) {
            if (t == 0 && ntiles > 0) {
                tile_iter(0, std::true_type{}, std::true_type{}, 0);
                t = 1;
            }
        }
        for (; t < ntiles; ++t) tile_iter(t, std::true_type{}, std::false_type{}, t % NB);
        if (item + (int)gridDim.x < nitems) load_q(item_of(item + (int)gridDim.x));

        // ---- O = O^T / l: lane holds d = 16dt + 4g + e of query li, and its query's full l.
        uint16_t* Oh = a.O + b * a.o_bs + h * a.o_hs;
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const float lt = lacc[t][0];
            const float inv = (lt > 0.f) ? 1.f / lt : 1.f;
            const int q = qw0 + t * 16 + li;
            if (q < a.seqQ) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 w = u32x2{pack2<kBf16>(o[t][dt][0] * inv, o[t][dt][1] * inv),
                                          pack2<kBf16>(o[t][dt][2] * inv, o[t][dt][3] * inv)};
                    *(u32x2*)(Oh + q * a.o_rs + dt * 16 + g * 4) = w;
                }
            }
        }
        __syncthreads();   // every wave is done with the LDS ring before the next item's copies
    }
}

// ---- fp32 arm on the matrix cores -------------------------------------------------------
// v_mfma_f32_16x16x4_f32 multiplies and accumulates in fp32. Lane L holds A[L % 16][L / 16],
// B[L / 16][L % 16] and C[4 (L / 16) + i][L % 16], i < 4 (cdna4::mfma::*_16x16x4f32 and its exact
// small-integer GEMM test). The reduction index of a product may be permuted freely as long as A
// and B agree, which gives every lane contiguous operands:
//   S^T = K Q^T, step s: lane (r = L % 16, g = L / 16) supplies K[key r][g D/4 + s] and
//                        Q[query r][g D/4 + s]; C: lane (r, g) holds keys 4g + i of query r.
//   O^T = V^T P^T, step s (keys 4g + s): B is the lane's own P of key 4g + s; A for row block b is
//                        V[key 4g + s][16 b + r]; C: lane (r, g) holds O[query r][16 b + 4 g + i].
// A workgroup of kF32Waves waves serves 16 queries of one (batch, head); wave w takes the 16-key
// chunks w, w + W, ... (the causal diagonal spreads over the waves), keeps a running base-2
// (m, l, O), and the waves merge through LDS at the end. The next chunk's K and V are loaded
// into registers while the current one is computed.
constexpr int kF32Br = 16;      // queries per workgroup
// Waves per workgroup: at the reference configuration (B1 H8 S512 D64, 256 workgroups) the
// per-wave chain of chunks bounds the time; eight waves ran 46.4 TFLOP/s against 43.8 with four
// and 41.6 with sixteen (the LDS merge grows).
constexpr int kF32Waves = 8;

template <int D>
__device__ __forceinline__ void f32_chunk_load(const float* __restrict__ Kh, const float* __restrict__ Vh, int kb,
                                               int seqK, int r, int g, float (&kf)[D / 4], float (&vf)[4][D / 16]) {
    constexpr int DS = D / 4;
    const float* kp = Kh + (size_t)min(kb + r, seqK - 1) * D + g * DS;
#pragma unroll
    for (int s = 0; s < DS; s += 4) {
        const float4 v = *(const float4*)(kp + s);
        kf[s] = v.x; kf[s + 1] = v.y; kf[s + 2] = v.z; kf[s + 3] = v.w;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float* vp = Vh + (size_t)min(kb + 4 * g + s, seqK - 1) * D + r;
#pragma unroll
        for (int b = 0; b < D / 16; ++b) vf[s][b] = vp[16 * b];
    }
}

template <int D>
__global__ __launch_bounds__(64 * kF32Waves) void fa_f32(const float* __restrict__ Q, const float* __restrict__ K,
                                                         const float* __restrict__ V, float* __restrict__ O, int seqQ,
                                                         int seqK, int nQH, int nKVH, int causal, int nqb, int xcd_map,
                                                         float sc) {
    constexpr int DS = D / 4, NB = D / 16;
    __shared__ __attribute__((aligned(16))) float o_s[kF32Waves][kF32Br][D];
    __shared__ float m_s[kF32Waves][kF32Br], l_s[kF32Waves][kF32Br];
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    int bh, qb;
    block_item(blockIdx.x, nqb, xcd_map, bh, qb);
    const int b = bh / nQH, h = bh % nQH;
    const int kvh = h / (nQH / nKVH);
    const int q0 = qb * kF32Br;
    const float* Qh = Q + ((size_t)b * nQH + h) * (size_t)seqQ * D;
    const float* Kh = K + ((size_t)b * nKVH + kvh) * (size_t)seqK * D;
    const float* Vh = V + ((size_t)b * nKVH + kvh) * (size_t)seqK * D;

    float qf[DS];
    {
        const float* qp = Qh + (size_t)min(q0 + r, seqQ - 1) * D + g * DS;
#pragma unroll
        for (int s = 0; s < DS; s += 4) {
            const float4 v = *(const float4*)(qp + s);
            qf[s] = v.x; qf[s + 1] = v.y; qf[s + 2] = v.z; qf[s + 3] = v.w;
        }
    }
    const int kend = causal ? min(seqK, q0 + kF32Br) : seqK;
    const int qrow = q0 + r;
    float m = kInitM, lpart = 0.f;
    f32x4 o[NB];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) o[bb] = f32x4{0.f, 0.f, 0.f, 0.f};

    float kf[DS], vf[4][NB];
    int kb = wave * 16;
    if (kb < kend) f32_chunk_load<D>(Kh, Vh, kb, seqK, r, g, kf, vf);
    for (; kb < kend; kb += 16 * kF32Waves) {
        f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < DS; ++s) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[s], qf[s], st, 0, 0, 0);
        float vc[4][NB];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) vc[s][bb] = vf[s][bb];
        const int kn = kb + 16 * kF32Waves;
        if (kn < kend) f32_chunk_load<D>(Kh, Vh, kn, seqK, r, g, kf, vf);   // next chunk, in flight
        float p[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = kb + 4 * g + i;
            p[i] = (key < kend && !(causal && key > qrow)) ? st[i] * sc : -INFINITY;
            mx = fmaxf(mx, p[i]);
        }
        mx = cross_row_allreduce(mx, Max{});
        const float mnew = fmaxf(m, mx);
        const float alpha = exp2f(m - mnew);
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = exp2f(p[i] - mnew);
            ps += p[i];
        }
        lpart = lpart * alpha + ps;
        m = mnew;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) o[bb] *= alpha;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) o[bb] = __builtin_amdgcn_mfma_f32_16x16x4f32(vc[s][bb], p[s], o[bb], 0, 0, 0);
    }
    const float l = cross_row_allreduce(lpart, Sum{});
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) *(f32x4*)&o_s[wave][r][16 * bb + 4 * g] = o[bb];
    if (g == 0) {
        m_s[wave][r] = m;
        l_s[wave][r] = l;
    }
    __syncthreads();
    float* Oh = O + ((size_t)b * nQH + h) * (size_t)seqQ * D;
    for (int idx = (int)threadIdx.x; idx < kF32Br * D; idx += 64 * kF32Waves) {
        const int q = idx / D, d = idx % D;
        if (q0 + q >= seqQ) break;
        float M = kInitM;
#pragma unroll
        for (int w = 0; w < kF32Waves; ++w) M = fmaxf(M, m_s[w][q]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < kF32Waves; ++w) {
            const float wt = exp2f(m_s[w][q] - M);
            L = fmaf(wt, l_s[w][q], L);
            acc = fmaf(wt, o_s[w][q][d], acc);
        }
        Oh[(size_t)(q0 + q) * D + d] = L > 0.f ? acc / L : 0.f;
    }
}

// ---- small problems: the keys of 16 queries split over the waves of a workgroup -------------
// When the regular grid has too few workgroups to fill the chip (e.g. the FA2 reference
// configuration: 8 heads x 512 queries), one workgroup of W waves serves 16 queries of one
// (batch, head): wave w streams the w-th contiguous part of the visible keys through its own LDS
// ring (the per-wave loop of the short-cache decode kernel, with the 16 queries as its columns and
// the causal mask), then the waves merge their (m, l, O) through LDS over their rings.
// Waves per workgroup: the LDS holds one two-stage K/V ring per wave (16 KiB per wave at D = 64,
// 32 KiB at D = 128), so the large form (128 KiB) allows one workgroup per CU and the small form
// two; the launcher takes the large form when one round of workgroups covers the grid.
template <int D> constexpr int small_waves(bool large) { return (D == 64 ? 8 : 4) / (large ? 1 : 2); }

template <int D, bool kBf16, int W>
__global__ __launch_bounds__(64 * W) void fa_small(PrefillArgs a) {
    constexpr int ND = D / 32, NDT = D / 16;
    constexpr int kStage = stream::kDecT * D;
    constexpr int kRing = stream::kDecStages * kStage;
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[W * kRing];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[W * kRing];
    static_assert((size_t)W * 16 * D * sizeof(float) <= sizeof(k_lds), "O partials fit over the K rings");
    static_assert((size_t)W * 16 * 2 * sizeof(float) <= sizeof(v_lds), "(m, l) partials fit over the V rings");

    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const int li = lane & 15, g = lane >> 4;
    const int nqb = (a.seqQ + 15) / 16;
    int bh, qblk;
    block_item(blockIdx.x, nqb, a.xcd_map, bh, qblk);
    const int b = bh / a.nQH, h = bh % a.nQH;
    const int kvh = h / (a.nQH / a.nKVH);
    const int q0 = qblk * 16;
    const int nrows = min(16, a.seqQ - q0);
    const uint16_t* Qh = a.Q + b * a.q_bs + h * a.q_hs;
    const uint16_t* Kh = a.K + b * a.k_bs + kvh * a.k_hs;
    const uint16_t* Vh = a.V + b * a.k_bs + kvh * a.k_hs;

    u32x4 qb[1][ND];
#pragma unroll
    for (int c = 0; c < ND; ++c) {
        qb[0][c] = u32x4{0u, 0u, 0u, 0u};
        if (li < nrows) qb[0][c] = *(const u32x4*)(Qh + (q0 + li) * a.q_rs + c * 32 + g * 8);
        asm volatile("" : : "v"(qb[0][c]));   // the loads complete before the first copy is issued
    }
    const int kend = a.causal ? min(a.seqK, q0 + 16) : a.seqK;
    const int kpw = ((kend + W - 1) / W + stream::kDecT - 1) / stream::kDecT * stream::kDecT;
    const int kbeg = min(kend, wave * kpw);
    const int kstop = min(kend, kbeg + kpw);
    f32x4 o[1][NDT], lacc[1];
    float m[1];
    stream::stream_keys<D, kBf16, stream::kDecStages>(Kh, Vh, a.k_rs, a.seqK, kbeg, kstop, q0, a.causal, a.sc, qb, o,
                                                      lacc, m, k_lds + wave * kRing, v_lds + wave * kRing, lane);
    __syncthreads();   // every wave is done with its ring: reuse the LDS for the partials
    float* po = (float*)k_lds;   // [W][16 queries][D]
    float* pml = (float*)v_lds;  // [W][16 queries][2]
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
        *(f32x4*)(po + ((size_t)wave * 16 + li) * D + dt * 16 + g * 4) = o[0][dt];
    if (g == 0) {
        pml[(wave * 16 + li) * 2] = m[0];
        pml[(wave * 16 + li) * 2 + 1] = lacc[0][0];
    }
    __syncthreads();
    uint16_t* Oh = a.O + b * a.o_bs + h * a.o_hs;
    for (int p = (int)threadIdx.x; p < nrows * (D / 2); p += 64 * W) {
        const int r = p / (D / 2), d = 2 * (p % (D / 2));
        float M = kInitM;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, pml[(w * 16 + r) * 2]);
        float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float wt = exp2f(pml[(w * 16 + r) * 2] - M);
            L = fmaf(wt, pml[(w * 16 + r) * 2 + 1], L);
            const float2 v = *(const float2*)(po + ((size_t)w * 16 + r) * D + d);
            o0 = fmaf(wt, v.x, o0);
            o1 = fmaf(wt, v.y, o1);
        }
        const float inv = L > 0.f ? 1.f / L : 1.f;
        *(uint32_t*)(Oh + (q0 + r) * a.o_rs + d) = pack2<kBf16>(o0 * inv, o1 * inv);
    }
}

// Kernel choice for the 16-bit path: the pipelined 8 waves x 32 queries (two waves per SIMD, one
// workgroup per CU) once its 256-query blocks fill the CUs at least once (causal) or a quarter of
// them (non-causal: every block has the same work, and one fast workgroup per block beat four-wave
// workgroups of 64 queries at every size measured down to 64 blocks, e.g. B1 H8 S4096 622 -> 705
// TFLOP/s; causal blocks below one round left the heaviest block on the critical path, e.g. B1 H12
// S4096 603 -> 547); 4 waves x 16 queries for the remaining mid-size causal problems; for problems
// whose 64-query blocks would not fill the CUs twice over, 16 queries per workgroup with the keys
// split over its waves (the large form when one round of workgroups covers the grid).
struct PrefillPlan { int kernel, waves, rows; long long grid; };

template <int D>
PrefillPlan plan_mfma(const cdna3_prefill_cfg& c) {
    const long long heads = (long long)c.batch * c.nQHeads;
    const int cus = device_cus();
    PrefillPlan p;
    const long long blocks8 = heads * ((c.seqQ + 255) / 256);
    if (blocks8 >= (c.causal ? cus : cus / 4)) {
        p.kernel = CDNA4_KERNEL_PREFILL_MFMA_8W; p.waves = 8; p.rows = 256;
        p.grid = blocks8;
        // One resident workgroup per CU at W = 8 (LDS and VGPRs allow no second), so a grid of one
        // workgroup per CU (a multiple of 8, see the item mapping) runs every item without
        // relaunch gaps between workgroups.
        const int pcus = cus & ~7;
        if (pcus >= 8 && p.grid > pcus) p.grid = pcus;
    } else if (heads * ((c.seqQ + 63) / 64) >= 2LL * cus) {
        p.kernel = CDNA4_KERNEL_PREFILL_MFMA_4W; p.waves = 4; p.rows = 64;
        p.grid = heads * ((c.seqQ + 63) / 64);
    } else {
        p.kernel = CDNA4_KERNEL_PREFILL_SMALL; p.rows = 16;
        p.grid = heads * ((c.seqQ + 15) / 16);
        p.waves = small_waves<D>(p.grid <= cus);
    }
    return p;
}

PrefillArgs make_args(const cdna3_prefill_cfg& c, const cdna3_prefill_strides& st, const void* Q, const void* K,
                      const void* V, void* O, int rows) {
    PrefillArgs a;
    a.Q = (const uint16_t*)Q; a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.O = (uint16_t*)O;
    a.q_bs = st.q_batch; a.q_hs = st.q_head; a.q_rs = st.q_row;
    a.k_bs = st.kv_batch; a.k_hs = st.kv_head; a.k_rs = st.kv_row;
    a.o_bs = st.o_batch; a.o_hs = st.o_head; a.o_rs = st.o_row;
    a.seqQ = c.seqQ; a.seqK = c.seqK; a.nQH = c.nQHeads; a.nKVH = c.nKVHeads; a.batch = c.batch;
    a.causal = c.causal ? 1 : 0;
    a.nqb = (c.seqQ + rows - 1) / rows;
    a.xcd_map = 0;
    a.copy32 = (long long)kBc * st.kv_row * 2 < (1LL << 32) ? 1 : 0;
    a.sc = kLog2e / sqrtf((float)c.D);
    return a;
}

template <int D, bool kBf16>
int dispatch_mfma(const cdna3_prefill_cfg& c, const cdna3_prefill_strides& st, const void* Q, const void* K,
                  const void* V, void* O, hipStream_t s) {
    const PrefillPlan p = plan_mfma<D>(c);
    PrefillArgs a = make_args(c, st, Q, K, V, O, p.rows);
    const long long nbh = (long long)c.batch * c.nQHeads;
    if (nbh * a.nqb > 0x7fffffffLL) return CDNA4_ERR_INVALID_VALUE;
    switch (p.kernel) {
        case CDNA4_KERNEL_PREFILL_MFMA_8W:
            a.xcd_map = (nbh % 8 == 0) ? 1 : 0;
            fa_pipe<D, 8, 2, kBf16><<<(unsigned)p.grid, 64 * 8, 0, s>>>(a);
            break;
        case CDNA4_KERNEL_PREFILL_MFMA_4W:
            a.xcd_map = (nbh % 8 == 0) ? 1 : 0;
            fa_mfma<D, 4, 1, kBf16><<<(unsigned)p.grid, 64 * 4, 0, s>>>(a);
            break;
        default:
            a.xcd_map = (nbh % 8 == 0) ? 1 : 0;
            if (p.waves == small_waves<D>(true))
                fa_small<D, kBf16, small_waves<D>(true)><<<(unsigned)p.grid, 64 * small_waves<D>(true), 0, s>>>(a);
            else
                fa_small<D, kBf16, small_waves<D>(false)><<<(unsigned)p.grid, 64 * small_waves<D>(false), 0, s>>>(a);
    }
    return launch_status();
}

int check_cfg(const cdna3_prefill_cfg* cfg, const void* Q, const void* K, const void* V, const void* O) {
    if (!cfg) return CDNA4_ERR_INVALID_VALUE;
    const cdna3_prefill_cfg& c = *cfg;
    if (c.D != 64 && c.D != 128) return CDNA4_ERR_INVALID_VALUE;
    if (c.seqQ < 1 || c.seqK < 1 || c.nQHeads < 1 || c.nKVHeads < 1 || c.batch < 1) return CDNA4_ERR_INVALID_VALUE;
    if (c.nQHeads % c.nKVHeads) return CDNA4_ERR_INVALID_VALUE;
    if (c.causal && c.seqQ != c.seqK) return CDNA4_ERR_INVALID_VALUE;
    if (!Q || !K || !V || !O) return CDNA4_ERR_INVALID_VALUE;
    return 0;
}

cdna3_prefill_strides contiguous_strides(const cdna3_prefill_cfg& c) {
    cdna3_prefill_strides st;
    st.q_row = st.kv_row = st.o_row = c.D;
    st.q_head = st.o_head = (long long)c.seqQ * c.D;
    st.kv_head = (long long)c.seqK * c.D;
    st.q_batch = st.o_batch = st.q_head * c.nQHeads;
    st.kv_batch = st.kv_head * c.nKVHeads;
    return st;
}

}  // namespace
}  // namespace cdna4

using namespace cdna4;

extern "C" int cdna3_attn_prefill(const void* Q, const void* K, const void* V, void* O, const cdna3_prefill_cfg* cfg,
                                  int dtype, cdna4_stream_t stream) {
    if (int e = check_cfg(cfg, Q, K, V, O)) return e;
    const cdna3_prefill_cfg& c = *cfg;
    if (dtype != CDNA4_F16 && dtype != CDNA4_BF16 && dtype != CDNA4_F32) return CDNA4_ERR_INVALID_VALUE;
    // 16-byte loads of Q, K, V rows (both kernels); O rows are stored 8 (16-bit) or 4 bytes at a time.
    if ((((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V) & 15u) || ((uintptr_t)O & (dtype == CDNA4_F32 ? 3u : 7u)))
        return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    if (dtype == CDNA4_F32) {
        const int nqb = (c.seqQ + kF32Br - 1) / kF32Br;
        const long long blocks = (long long)c.batch * c.nQHeads * nqb;
        if (blocks > 0x7fffffffLL) return CDNA4_ERR_INVALID_VALUE;
        const float sc = kLog2e / sqrtf((float)c.D);
        const int xcd = ((long long)c.batch * c.nQHeads % 8 == 0) ? 1 : 0;
        if (c.D == 128)
            fa_f32<128><<<(unsigned)blocks, 64 * kF32Waves, 0, s>>>((const float*)Q, (const float*)K, (const float*)V,
                                                                    (float*)O, c.seqQ, c.seqK, c.nQHeads, c.nKVHeads,
                                                                    c.causal ? 1 : 0, nqb, xcd, sc);
        else
            fa_f32<64><<<(unsigned)blocks, 64 * kF32Waves, 0, s>>>((const float*)Q, (const float*)K, (const float*)V,
                                                                   (float*)O, c.seqQ, c.seqK, c.nQHeads, c.nKVHeads,
                                                                   c.causal ? 1 : 0, nqb, xcd, sc);
        return launch_status();
    }
    const cdna3_prefill_strides st = contiguous_strides(c);
    const bool bf = dtype == CDNA4_BF16;
    if (c.D == 128)
        return bf ? dispatch_mfma<128, true>(c, st, Q, K, V, O, s) : dispatch_mfma<128, false>(c, st, Q, K, V, O, s);
    return bf ? dispatch_mfma<64, true>(c, st, Q, K, V, O, s) : dispatch_mfma<64, false>(c, st, Q, K, V, O, s);
}

extern "C" int cdna3_attn_prefill_strided(const void* Q, const void* K, const void* V, void* O,
                                          const cdna3_prefill_cfg* cfg, const cdna3_prefill_strides* strides,
                                          int dtype, cdna4_stream_t stream) {
    if (int e = check_cfg(cfg, Q, K, V, O)) return e;
    if (!strides) return CDNA4_ERR_INVALID_VALUE;
    const cdna3_prefill_cfg& c = *cfg;
    const cdna3_prefill_strides& st = *strides;
    if (dtype != CDNA4_F16 && dtype != CDNA4_BF16) return CDNA4_ERR_INVALID_VALUE;
    // 16-byte row loads of Q, K, V and 8-byte stores of O: every stride a multiple of 8 (4 for O)
    // elements, rows no shorter than D.
    const long long in[6] = {st.q_batch, st.q_head, st.q_row, st.kv_batch, st.kv_head, st.kv_row};
    for (long long x : in)
        if (x < 0 || (x & 7)) return CDNA4_ERR_INVALID_VALUE;
    const long long out[3] = {st.o_batch, st.o_head, st.o_row};
    for (long long x : out)
        if (x < 0 || (x & 3)) return CDNA4_ERR_INVALID_VALUE;
    if (st.q_row < c.D || st.kv_row < c.D || st.o_row < c.D) return CDNA4_ERR_INVALID_VALUE;
    if ((((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V) & 15u) || ((uintptr_t)O & 7u)) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    const bool bf = dtype == CDNA4_BF16;
    if (c.D == 128)
        return bf ? dispatch_mfma<128, true>(c, st, Q, K, V, O, s) : dispatch_mfma<128, false>(c, st, Q, K, V, O, s);
    return bf ? dispatch_mfma<64, true>(c, st, Q, K, V, O, s) : dispatch_mfma<64, false>(c, st, Q, K, V, O, s);
}

extern "C" int cdna3_attn_prefill_plan(const cdna3_prefill_cfg* cfg, int dtype, cdna3_plan_info* out) {
    if (!cfg || !out) return CDNA4_ERR_INVALID_VALUE;
    const cdna3_prefill_cfg& c = *cfg;
    if (c.D != 64 && c.D != 128) return CDNA4_ERR_INVALID_VALUE;
    if (c.seqQ < 1 || c.seqK < 1 || c.nQHeads < 1 || c.nKVHeads < 1 || c.batch < 1) return CDNA4_ERR_INVALID_VALUE;
    if (c.nQHeads % c.nKVHeads || (c.causal && c.seqQ != c.seqK)) return CDNA4_ERR_INVALID_VALUE;
    if (dtype == CDNA4_F32) {
        out->kernel = CDNA4_KERNEL_PREFILL_F32;
        out->waves = kF32Waves;
        out->rows = kF32Br;
        out->grid = (long long)c.batch * c.nQHeads * ((c.seqQ + kF32Br - 1) / kF32Br);
    } else if (dtype == CDNA4_F16 || dtype == CDNA4_BF16) {
        const PrefillPlan p = c.D == 128 ? plan_mfma<128>(c) : plan_mfma<64>(c);
        out->kernel = p.kernel;
        out->waves = p.waves;
        out->rows = p.rows;
        out->grid = p.grid;
    } else {
        return CDNA4_ERR_INVALID_VALUE;
    }
    out->partials = 1;
    out->workspace = 0;
    return 0;
}
