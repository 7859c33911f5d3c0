// Prompt-path GEMM of the small-LLM runtime (gfx950): Y[M][N] (+)= X[M][K] W[N][K]^T with fp16
// X and W (both row-major, K contiguous), fp32 accumulation, fp32 or fp16 Y.
//
// Reference behaviour restated: the reference runs these products through rocBLAS gemm_ex
// (cdna3-prims/include/cdna3/runtime/rocblas_gemm.hpp:8-20; forward.hpp:70-131), Y = X W^T with W
// the [out][in] weight as the model files hold it, beta 0 (Q|K|V, gate|up) or 1 (the O and down
// projections added into the fp32 residual).
//
// MI355X design: at prompt lengths of a few hundred tokens these GEMMs are small (0.6-4.8 GFLOP,
// 2-10 MB of operands) and a launch is over in a few microseconds, so what sets the time is how
// many workgroups the grid gives each CU and how many bytes each CU keeps in flight. The tile
// (BM x BN, from a small menu) is chosen per shape so that the grid is about one round of one
// workgroup per CU, and each workgroup streams 64-wide K stages of both operand tiles HBM -> LDS
// with asynchronous copies (global_load_lds_dwordx4) into a ring of S stages, S - 1 ahead of the
// stage being multiplied (S as deep as 128 KB of LDS allows, up to 8). Four waves compute Y^T =
// W X^T on v_mfma_f32_16x16x32_f16: W rows are the A operand, X rows the B operand.
//
// LDS layout (the prefill's K tile at D = 64, whose reads were measured free of bank conflicts):
// a stage holds BN rows of W then BM rows of X, 128 bytes per row; 16-byte chunk c of row r sits
// at position c ^ swz_k<64>(r % 32). An operand block (16 rows) of 32-row group G is read in the
// permuted row order 32 G + 8 (l / 4) + l % 4 + 4 u (A-row / B-column l, u = 0 or 1): the lanes
// of one read then touch every bank once, and a lane's four accumulator values are four
// consecutive output columns n (one 16-byte or 8-byte store). Wave (wm, wn) takes block u = wn of
// every W group and u = wm of every X group of the tile. Rows past M or N read the last valid row
// (their results are not stored).
#include "attn_stream.hpp"

namespace cdna4 {
namespace {

typedef _Float16 gf16x8 __attribute__((ext_vector_type(8)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 gf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;        // K per stage (one 128-byte LDS row per operand row)
constexpr int kKMul = kBK;     // K must be a multiple of this
constexpr int kRowBytes = kBK * 2;
constexpr int kLdsBudget = 128 * 1024;

// Ring depth for a BM x BN tile: as many stages as the LDS budget holds, at most 8.
constexpr int ring_stages(int bm, int bn, int budget = kLdsBudget) {
    const int s = budget / ((bm + bn) * kRowBytes);
    return s > 8 ? 8 : s;
}

// Wait until at most `younger` stages' copies (kPerStage each per wave) are still in flight.
template <int kPerStage, int S>
__device__ __forceinline__ void wait_stages(int younger) {
    static_assert(S >= 2 && S <= 12 && (S - 2) * kPerStage <= 63, "ring depth within the vmcnt range");
#define CDNA4_GEMM_WAIT(y) \
    case y: asm volatile("s_waitcnt vmcnt(%0)" : : "n"((y) * kPerStage) : "memory"); break;
    switch (younger) {
        CDNA4_GEMM_WAIT(0) CDNA4_GEMM_WAIT(1) CDNA4_GEMM_WAIT(2) CDNA4_GEMM_WAIT(3)
        CDNA4_GEMM_WAIT(4) CDNA4_GEMM_WAIT(5) CDNA4_GEMM_WAIT(6) CDNA4_GEMM_WAIT(7)
        CDNA4_GEMM_WAIT(8) CDNA4_GEMM_WAIT(9) CDNA4_GEMM_WAIT(10)
        default: asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); break;
    }
#undef CDNA4_GEMM_WAIT
}

// Tile of workgroup b in a grid of tm x tn tiles (1-D). Workgroups go to the 8 XCDs round-robin
// (XCD = b % 8); when tn is a multiple of 8, XCD x takes the n tiles x tn/8 .. (x+1) tn/8 - 1 with
// every m tile (m fastest), so each W row is fetched into one XCD's L2 only and re-read there by
// that XCD's tiles, and X (the smaller operand at prompt lengths) is what each XCD fetches whole.
__device__ __forceinline__ void tile_of(int b, int tm, int tn, int& mt, int& nt) {
    if ((tn & 7) == 0) {
        const int x = b & 7, s = b >> 3;
        mt = s % tm;
        nt = x * (tn >> 3) + s / tm;
    } else {
        mt = b % tm;
        nt = b / tm;
    }
}

// Output forms: fp16 or fp32 Y (Y = X W^T, + Y with kAccum), or the SiLU-gated product of the
// SwiGLU MLP (kSilu): W holds 2F rows, gate rows 0 .. F - 1 then up rows F .. 2F - 1, and Y [M][F]
// fp16 = fp16(silu(X Wg^T) * (X Wu^T)) in fp32, the rounding the separate silu_mul kernel applies
// to the fp32 product. A kSilu tile of BN rows takes BN / 2 gate rows and the BN / 2 up rows of the
// same output columns, so a lane holds both values of its columns.
enum { kOutF16 = 0, kOutF32 = 1, kOutSilu = 2, kOutQKV = 3 };

// LDS budget of a tile's ring. The Q|K|V epilogue's 64 x 64 tiles take 64 KiB (four stages), so
// two workgroups share a CU: at config 5 (512 x 2304 x 768) that ran the projection + append in a
// time to first token of 0.770 ms against 0.804 with eight stages and one workgroup per CU, and
// 0.788 with the 64 x 128 tile.
// 64 x 32 tiles (the runtime's residual projections, llm_gemm_f16 with cold operands) likewise
// take 64 KiB (five stages), two workgroups per CU.
constexpr int ring_budget(int kOut, int bm, int bn) {
    return (kOut == kOutQKV && bm + bn <= 128) || (bm == 64 && bn == 32) ? 64 * 1024 : kLdsBudget;
}

// kOutQKV: the prompt's Q|K|V projection (columns [0, QD) query heads, [QD, QD + KVD) key heads,
// the rest value heads, D columns each) with the runtime's RoPE + append in the epilogue: each
// value is rounded to fp16 as the projection's output, the (d, d + D/2) pairs of query and key
// heads rotated with the cos/sin rows of positions pos0 + m (rope_pair, as the separate append
// kernel does), queries written head-major to q_out [QD / D][T][D] and keys and values into the
// caches [heads][max_seq][D] at row pos0 + m. Tiles are whole heads (BN % D == 0), so a lane holds
// both columns of its pairs: block i and block i + D / 64 (32 columns per block).

template <int BM, int BN, int kOut, bool kAccum>
__global__ __launch_bounds__(256) void gemm_ring(const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                                                 void* __restrict__ Y, int M, int N, int K, int ldy, QkvOut qe) {
    static_assert(BM % 32 == 0 && BN % 32 == 0, "tiles are whole 32-row groups");
    static_assert(kOut != kOutSilu || (BN % 64 == 0 && !kAccum), "a SiLU tile pairs whole gate and up groups");
    constexpr bool kSilu = kOut == kOutSilu;
    constexpr int kTileCols = kSilu ? BN / 2 : BN;   // output columns per tile
    const int ncols = kSilu ? N / 2 : N;              // output columns (F for kSilu)
    constexpr int S = ring_stages(BM, BN, ring_budget(kOut, BM, BN));
    constexpr int FM = BM / 32, FN = BN / 32;        // 16-row blocks per wave: X (m), W (n)
    constexpr int kStage = (BN + BM) * kRowBytes;    // bytes per ring stage
    constexpr int kCopies = (BN + BM) / 8;           // 1 KB copy instructions per stage
    constexpr int kCopiesW = kCopies / 4;            // per wave
    static_assert(kCopies % 4 == 0, "copies split evenly over the four waves");
    __shared__ __attribute__((aligned(16))) char lds[S * kStage];

    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int li = lane & 15, g = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    int mt, nt;
    tile_of((int)blockIdx.x, (M + BM - 1) / BM, (ncols + kTileCols - 1) / kTileCols, mt, nt);
    const int m0 = mt * BM, n0 = nt * kTileCols;

    // Copy j of this wave is instruction c = wave + 4 j of a stage: its lane l fills LDS row
    // 8 c + l / 8 at chunk position l % 8 (1 KB of the stage at byte 1024 c) from global chunk
    // (l % 8) ^ swz(row) of W row n0 + row (rows below BN) or X row m0 + row - BN; whether the
    // instruction copies W or X is uniform over the wave.
    uint32_t coff[kCopiesW];
    bool cw[kCopiesW];
#pragma unroll
    for (int j = 0; j < kCopiesW; ++j) {
        const int c = wave + 4 * j;
        const int row = c * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ tile::swz_k<64>(row & 31);
        cw[j] = c * 8 < BN;
        int r;
        if (!cw[j]) r = min(m0 + row - BN, M - 1);
        else if (kSilu) r = row < BN / 2 ? min(n0 + row, ncols - 1) : ncols + min(n0 + row - BN / 2, ncols - 1);
        else r = min(n0 + row, N - 1);
        coff[j] = (uint32_t)r * (uint32_t)K * 2u + (uint32_t)chunk * 16u;
    }
    auto issue = [&](int kt, int buf) {   // the copies of stage kt (k0 = 64 kt) into ring slot buf
        const uint16_t* wk = W + (size_t)kt * kBK;
        const uint16_t* xk = X + (size_t)kt * kBK;
#pragma unroll
        for (int j = 0; j < kCopiesW; ++j)
            stream::dma16_s(cw[j] ? wk : xk, coff[j], lds + buf * kStage + (wave + 4 * j) * 1024);
    };

    // Operand reads: W block i (group i, u = wn), X block j (group j, u = wm); K step kc of a stage
    // flips bit 6 (chunk c -> c + 4).
    const int r0 = 8 * (li >> 2) + (li & 3);
    const uint32_t rd = (uint32_t)(r0 * kRowBytes + ((g ^ tile::swz_k<64>(r0)) * 16));
    const uint32_t rw = rd + (uint32_t)wn * 512u;
    const uint32_t rx = (uint32_t)BN * kRowBytes + rd + (uint32_t)wm * 512u;

    gf32x4 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = gf32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = K / kBK;
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
        if (st < nk) issue(st, st);
    for (int kt = 0; kt < nk; ++kt) {
        // stage kt landed (this wave's copies; the barrier: every wave's), and every wave is past
        // stage kt - 1, whose slot now receives stage kt + S - 1
        wait_stages<kCopiesW, S>(min(S - 2, nk - 1 - kt));
        __syncthreads();
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        const char* st = lds + (kt % S) * kStage;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const uint32_t flip = (uint32_t)kc * 64u;
            u32x4 a[FN], b[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i) a[i] = *(const u32x4*)(st + ((rw + (uint32_t)i * 4096u) ^ flip));
#pragma unroll
            for (int j = 0; j < FM; ++j) b[j] = *(const u32x4*)(st + ((rx + (uint32_t)j * 4096u) ^ flip));
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(gf16x8, a[i]),
                                                                       __builtin_bit_cast(gf16x8, b[j]), acc[i][j], 0,
                                                                       0, 0);
        }
    }

    // acc[i][j] lane (li, g): Y[m][n .. n + 3], m = m0 + 32 j + r0 + 4 wm, n = n0 + 32 i + 8 g + 4 wn
    // (kSilu: gate group i < FN / 2 and up group i + FN / 2 hold the same columns n).
    if constexpr (kOut == kOutQKV) {
        const int hb = qe.D / 64;   // blocks per half head
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int m = m0 + 32 * j + r0 + 4 * wm;
            if (m >= M) continue;
            const float* cr = qe.cosv + (size_t)(qe.pos0 + m) * qe.D;
            const float* sr = qe.sinv + (size_t)(qe.pos0 + m) * qe.D;
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                if ((i / hb) % 2) continue;   // block i in the second half of its head: done with its partner
                const int n = n0 + 32 * i + 8 * g + 4 * wn;   // a first-half column; n + D / 2 its partner
                if (n >= ncols) continue;
                const int d = n % qe.D, half = qe.D / 2;
                const gf32x4 va = acc[i][j], vb = acc[(i + hb) % FN][j];
                uint32_t lo[4], hi[4];
                uint16_t* dst;
                if (n < qe.QD + qe.KVD) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        rope_pair(f32_to_f16_bits(va[e]), f32_to_f16_bits(vb[e]), cr[d + e], sr[d + e],
                                  cr[d + e + half], sr[d + e + half], lo[e], hi[e]);
                    dst = n < qe.QD ? qe.q_out + ((size_t)(n / qe.D) * qe.T + m) * qe.D
                                    : qe.Kc + ((size_t)((n - qe.QD) / qe.D) * qe.max_seq + qe.pos0 + m) * qe.D;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = f32_to_f16_bits(va[e]);
                        hi[e] = f32_to_f16_bits(vb[e]);
                    }
                    dst = qe.Vc + ((size_t)((n - qe.QD - qe.KVD) / qe.D) * qe.max_seq + qe.pos0 + m) * qe.D;
                }
                *(u32x2*)(dst + d) = u32x2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
                *(u32x2*)(dst + d + half) = u32x2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int m = m0 + 32 * j + r0 + 4 * wm;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < (kSilu ? FN / 2 : FN); ++i) {
            const int n = n0 + 32 * i + 8 * g + 4 * wn;
            if (n >= ncols) continue;
            gf32x4 v = acc[i][j];
            if constexpr (kSilu) {
                const gf32x4 u = acc[i + FN / 2][j];
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = f32_to_f16_bits(v[e] / (1.f + expf(-v[e])) * u[e]);
                *(u32x2*)((uint16_t*)Y + (size_t)m * ldy + n) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            } else if constexpr (kOut == kOutF32) {
                float* y = (float*)Y + (size_t)m * ldy + n;
                if constexpr (kAccum) v += *(const gf32x4*)y;
                *(gf32x4*)y = v;
            } else {
                _Float16* y = (_Float16*)Y + (size_t)m * ldy + n;
                if constexpr (kAccum) {
                    const gf16x4 o = *(const gf16x4*)y;
                    v += gf32x4{(float)o[0], (float)o[1], (float)o[2], (float)o[3]};
                }
                *(gf16x4*)y = gf16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            }
        }
    }
}

template <int BM, int BN>
int gemm_launch(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, bool accum, int M, int N, int K, int ldy,
                hipStream_t s) {
    const unsigned grid = ceil_div((size_t)M, BM) * ceil_div((size_t)N, BN);
    if (y_f32) {
        if (accum) gemm_ring<BM, BN, kOutF32, true><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy, QkvOut{});
        else gemm_ring<BM, BN, kOutF32, false><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy, QkvOut{});
    } else {
        if (accum) gemm_ring<BM, BN, kOutF16, true><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy, QkvOut{});
        else gemm_ring<BM, BN, kOutF16, false><<<grid, 256, 0, s>>>(X, W, Y, M, N, K, ldy, QkvOut{});
    }
    return launch_status();
}

template <int BM, int BN>
int gemm_silu_launch(const uint16_t* X, const uint16_t* W, void* Y, int M, int F, int K, int ldy, hipStream_t s) {
    const unsigned grid = ceil_div((size_t)M, BM) * ceil_div((size_t)F, BN / 2);
    gemm_ring<BM, BN, kOutSilu, false><<<grid, 256, 0, s>>>(X, W, Y, M, 2 * F, K, ldy, QkvOut{});
    return launch_status();
}

// The tile menu, and the estimate the dispatcher ranks it by: rounds of workgroups over the CUs
// (two workgroups per CU when the ring leaves room for a second in the 160 KB of LDS) times one
// workgroup's time: a fixed cost per K stage (the copy round trip the ring does not hide) plus its
// operand bytes at a per-CU stream rate and its MFMA work at a per-CU matrix rate. Calibrated on
// the cfg5 prompt shapes, where it picks the fastest tile of the menu measured on the box (Q|K|V
// 64 x 96: 7.7 us; O 32 x 32: 5.7; gate|up 128 x 96: 11.5; down 32 x 32: 13.6, event-timed).
struct Tile { int bm, bn; };
constexpr Tile kTiles[] = {{32, 32}, {64, 64}, {64, 96}, {64, 128}, {128, 64}, {128, 96}, {128, 128}};
constexpr double kStageUs = 0.1;           // per 64-wide K stage
constexpr double kCuBytesPerUs = 2.0e5;    // ~200 GB/s of operand tiles per CU
constexpr double kCuFlopsPerUs = 8.0e6;    // ~8 TFLOP/s of fp16 MFMA per CU

Tile pick_tile(int M, int N, int K, int cus, bool silu = false) {
    Tile best = {0, 0};
    double best_t = 1e300;
    for (const Tile& t : kTiles) {
        if (silu && t.bn % 64) continue;   // a SiLU tile pairs whole gate and up groups
        const int lds = ring_stages(t.bm, t.bn) * (t.bm + t.bn) * kRowBytes;
        const int per_cu = (160 * 1024) / lds >= 2 ? 2 : 1;
        const double tiles = (double)ceil_div((size_t)M, t.bm) * ceil_div((size_t)N, t.bn);
        const double rounds = ceil(tiles / ((double)cus * per_cu));
        const double wg = (double)(K / kBK) * kStageUs + (double)(t.bm + t.bn) * K * 2 / kCuBytesPerUs +
                          2.0 * t.bm * t.bn * K / kCuFlopsPerUs;
        const double est = rounds * wg;
        if (est < best_t) {
            best_t = est;
            best = t;
        }
    }
    return best;
}

}  // namespace

// Returns -1, launching nothing, for a shape this kernel does not take (K not a multiple of 64,
// N or ldy not a multiple of 4, X / W not 16-byte or Y not 16- (fp32) / 8-byte (fp16) aligned,
// operands past 4 GiB); the caller then uses rocBLAS. Otherwise 0 or the launch's error.
// cold: the operands arrive from HBM or the Infinity Cache, not L2 (the runtime's prompt, where
// each GEMM reads the previous kernel's output and a layer's weights once). There a 32 x 32 pick
// becomes 64 x 32 (half the W re-reads, five-stage ring, two workgroups per CU): at config 5 the
// O and down projections took the time to first token from 0.767 to 0.733 ms, though launched
// back to back on the same operands (all in L2) 64 x 32 ran no faster (O 5.9 against 6.0 us,
// down 14.1 against 13.7).
int llm_gemm_f16(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, bool accum, int M, int N, int K, int ldy,
                 hipStream_t s, bool cold) {
    if (M <= 0 || N <= 0 || K <= 0 || K % kKMul || N % 4 || ldy % 4 || ldy < N) return -1;
    if (((uintptr_t)X | (uintptr_t)W) % 16 || (uintptr_t)Y % (y_f32 ? 16 : 8)) return -1;
    if ((uint64_t)M * K * 2 >= (1ull << 32) || (uint64_t)N * K * 2 >= (1ull << 32)) return -1;   // 32-bit copy offsets
    const int cus = device_cus() > 0 ? device_cus() : 256;
    Tile t = pick_tile(M, N, K, cus);
    if (cold && t.bm == 32 && t.bn == 32 && M >= 64 &&
        (double)ceil_div((size_t)M, 64) * ceil_div((size_t)N, 32) <= 2.0 * cus)
        t = Tile{64, 32};
#define CDNA4_GEMM_TILE(a, b) \
    if (t.bm == a && t.bn == b) return gemm_launch<a, b>(X, W, Y, y_f32, accum, M, N, K, ldy, s);
    CDNA4_GEMM_TILE(32, 32) CDNA4_GEMM_TILE(64, 32) CDNA4_GEMM_TILE(64, 64) CDNA4_GEMM_TILE(64, 96)
    CDNA4_GEMM_TILE(64, 128) CDNA4_GEMM_TILE(128, 64) CDNA4_GEMM_TILE(128, 96) CDNA4_GEMM_TILE(128, 128)
#undef CDNA4_GEMM_TILE
    return -1;
}

// The prompt's Q|K|V projection X [M][K] x W [QD + 2 KVD][K]^T with the RoPE + append epilogue
// (kOutQKV; q_out, K and V caches as QkvOut describes, cos/sin tables [max_seq][D]). Tiles of
// whole heads only (BN % D == 0, D % 64 == 0): the tile of the single-pass menu with the least
// estimate among those. Returns -1, launching nothing, for shapes it does not take (the runtime
// then projects with llm_gemm_f16 and appends separately).
int llm_gemm_qkv_rope(const uint16_t* X, const uint16_t* W, int M, int K, const QkvOut& qe, hipStream_t s) {
    const int N = qe.QD + 2 * qe.KVD;
    if (M <= 0 || K <= 0 || K % kKMul || qe.D % 64 || qe.QD % qe.D || qe.KVD % qe.D) return -1;
    if (((uintptr_t)X | (uintptr_t)W) % 16 || ((uintptr_t)qe.q_out | (uintptr_t)qe.Kc | (uintptr_t)qe.Vc) % 8) return -1;
    if ((uint64_t)M * K * 2 >= (1ull << 32) || (uint64_t)N * K * 2 >= (1ull << 32)) return -1;
    const int cus = device_cus() > 0 ? device_cus() : 256;
    Tile best = {0, 0};
    double best_t = 1e300;
    for (const Tile& t : kTiles) {
        if (t.bn % qe.D || t.bn % 64) continue;
        const int lds = ring_stages(t.bm, t.bn, ring_budget(kOutQKV, t.bm, t.bn)) * (t.bm + t.bn) * kRowBytes;
        const int per_cu = (160 * 1024) / lds >= 2 ? 2 : 1;
        const double tiles = (double)ceil_div((size_t)M, t.bm) * ceil_div((size_t)N, t.bn);
        const double wg = (double)(K / kBK) * kStageUs + (double)(t.bm + t.bn) * K * 2 / kCuBytesPerUs +
                          2.0 * t.bm * t.bn * K / kCuFlopsPerUs;
        const double est = ceil(tiles / ((double)cus * per_cu)) * wg;
        if (est < best_t) {
            best_t = est;
            best = t;
        }
    }
    const unsigned grid = ceil_div((size_t)M, best.bm) * ceil_div((size_t)N, best.bn);
#define CDNA4_QKV_TILE(a, b)                                                                              \
    if (best.bm == a && best.bn == b) {                                                                     \
        gemm_ring<a, b, kOutQKV, false><<<grid, 256, 0, s>>>(X, W, nullptr, M, N, K, N, qe);                \
        return launch_status();                                                                             \
    }
    CDNA4_QKV_TILE(64, 64) CDNA4_QKV_TILE(64, 128) CDNA4_QKV_TILE(128, 64) CDNA4_QKV_TILE(128, 128)
#undef CDNA4_QKV_TILE
    return -1;
}

// Y[M][F] fp16 = fp16(silu(X Wg^T) * (X Wu^T)), W = [Wg; Wu] fp16 [2F][K] (the SwiGLU gate|up
// product followed by the SiLU product in one launch). Returns -1, launching nothing, for a shape
// the kernel does not take (as llm_gemm_f16; F a multiple of 4, Y 8-byte aligned).
int llm_gemm_f16_silu(const uint16_t* X, const uint16_t* W, void* Y, int M, int F, int K, int ldy, hipStream_t s) {
    if (M <= 0 || F <= 0 || K <= 0 || K % kKMul || F % 4 || ldy % 4 || ldy < F) return -1;
    if (((uintptr_t)X | (uintptr_t)W) % 16 || (uintptr_t)Y % 8) return -1;
    if ((uint64_t)M * K * 2 >= (1ull << 32) || (uint64_t)2 * F * K * 2 >= (1ull << 32)) return -1;
    const Tile t = pick_tile(M, 2 * F, K, device_cus() > 0 ? device_cus() : 256, true);
#define CDNA4_GEMM_TILE(a, b) \
    if (t.bm == a && t.bn == b) return gemm_silu_launch<a, b>(X, W, Y, M, F, K, ldy, s);
    CDNA4_GEMM_TILE(64, 64) CDNA4_GEMM_TILE(64, 128) CDNA4_GEMM_TILE(128, 64) CDNA4_GEMM_TILE(128, 128)
#undef CDNA4_GEMM_TILE
    return -1;
}

}  // namespace cdna4

extern "C" int cdna4_gemm_f16_nt_silu(const void* X, const void* W, void* Y, int M, int F, int K, int ldy,
                                      cdna4_stream_t stream) {
    if (M < 0 || F < 0 || K < 0) return CDNA4_ERR_INVALID_VALUE;
    if (M == 0 || F == 0) return 0;
    if (!X || !W || !Y) return CDNA4_ERR_INVALID_VALUE;
    if (int e = cdna4::check_device()) return e;
    const int e = cdna4::llm_gemm_f16_silu((const uint16_t*)X, (const uint16_t*)W, Y, M, F, K, ldy, (hipStream_t)stream);
    return e == -1 ? CDNA4_ERR_INVALID_VALUE : e;
}

extern "C" int cdna4_gemm_f16_nt_silu_tile(int M, int F, int K, int* bm, int* bn) {
    if (M <= 0 || F <= 0 || K <= 0 || !bm || !bn) return CDNA4_ERR_INVALID_VALUE;
    const cdna4::Tile t = cdna4::pick_tile(M, 2 * F, K, cdna4::device_cus() > 0 ? cdna4::device_cus() : 256, true);
    *bm = t.bm;
    *bn = t.bn;
    return 0;
}

extern "C" int cdna4_gemm_f16_nt_tile(int M, int N, int K, int* bm, int* bn) {
    if (M <= 0 || N <= 0 || K <= 0 || !bm || !bn) return CDNA4_ERR_INVALID_VALUE;
    const cdna4::Tile t = cdna4::pick_tile(M, N, K, cdna4::device_cus() > 0 ? cdna4::device_cus() : 256);
    *bm = t.bm;
    *bn = t.bn;
    return 0;
}

extern "C" int cdna4_gemm_f16_nt(const void* X, const void* W, void* Y, int y_f32, int accum, int M, int N, int K,
                                 int ldy, cdna4_stream_t stream) {
    if (M < 0 || N < 0 || K < 0 || (y_f32 != 0 && y_f32 != 1) || (accum != 0 && accum != 1))
        return CDNA4_ERR_INVALID_VALUE;
    if (M == 0 || N == 0) return 0;
    if (!X || !W || !Y) return CDNA4_ERR_INVALID_VALUE;
    if (int e = cdna4::check_device()) return e;
    const int e = cdna4::llm_gemm_f16((const uint16_t*)X, (const uint16_t*)W, Y, y_f32 == 1, accum == 1, M, N, K, ldy,
                                      (hipStream_t)stream, false);
    return e == -1 ? CDNA4_ERR_INVALID_VALUE : e;
}
