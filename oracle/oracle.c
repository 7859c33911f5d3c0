/*
 * oracle.c — CPU restatement of the reference's algorithms for the attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for libcdna4_attn.so: only the tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and never as the thing
 * that is measured or shipped. The product path never calls into it.
 *
 * Built as oracle/liboracle.so by oracle/Makefile (gcc, no GPU, no ROCm). Single-threaded,
 * plain C99, no FMA contraction (the x86-64 baseline target has none), so the attention
 * functions reproduce the reference's fp32 CPU references operation for operation.
 *
 * What each function follows (paths relative to the reference repository):
 *   orc_prefill_f32   cdna3-prims/tests/validate_attention_api.hip:27-51 (cpu_prefill)
 *   orc_prefill_rows  same arithmetic as orc_prefill_f32, for a list of (b, h, q) rows
 *   orc_decode_f32    cdna3-prims/tests/validate_attention_api.hip:53-72 (cpu_decode), with a
 *                     batch dimension and the strided cache of
 *                     cdna3-prims/include/cdna3/detail/fa_decode_dme_kernel.hpp:83-86
 *   orc_reduce        wave::dpp::reduce_{sum,max,min} semantics (research/wave-primitives/
 *                     include/wave_primitives/wave_reduce_dpp.hpp:101-108) over a whole array
 *   orc_scan_inclusive wave::dpp::scan_inclusive_* semantics (wave_scan_dpp.hpp:51-70)
 *   orc_rmsnorm_f32   cdna3-prims/include/cdna3/runtime/forward.hpp:34-56
 *   orc_layernorm_f32 research/wave-primitives/benchmarks/bench_layernorm.hip:51-114
 *   orc_softmax_rows_f32 research/wave-primitives/benchmarks/bench_softmax.hip:59-105
 *                     (softmax_kernel: row max, exp(x - max), row sum, x 1/sum), statistics in double
 *   orc_rope_table    cdna3-prims/include/cdna3/runtime/session.hpp:120-135 (fill_rope)
 *   orc_rope_f16      cdna3-prims/include/cdna3/runtime/forward.hpp:135-148 (rope_kernel),
 *                     reading every input element before any is written
 *   orc_scatter_kv_f16 cdna3-prims/include/cdna3/runtime/forward.hpp:209-220 (scatter_kv_kernel)
 *   orc_repack_f16    cdna3-prims/include/cdna3/runtime/forward.hpp:190-205 (repack_kernel)
 *   orc_rope_append_kv_f16  the layer-loop sequence of cdna3-prims/include/cdna3/runtime/
 *                     session.hpp:170-199: rope_kernel on Q and K, repack of Q to head-major,
 *                     scatter_kv_kernel of K and V into the cache at pos0
 *   generators        splitmix64 (Steele, Lea, Flood 2014), counter-based; Box-Muller normals
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- generators ------------------------------------------------------------------------ */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* i-th output of the splitmix64 stream seeded with `seed` (i = 0, 1, ...). */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * 0x9e3779b97f4a7c15ULL);
}

/* Uniform double in [0, 1) from the top 53 bits. */
static double u01(uint64_t x) { return (double)(x >> 11) * (1.0 / 9007199254740992.0); }

void orc_fill_uniform_f32(uint64_t seed, size_t n, float lo, float hi, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)(lo + (hi - lo) * u01(orc_splitmix64_at(seed, i)));
}

void orc_fill_uniform_f64(uint64_t seed, size_t n, double lo, double hi, double* out) {
    for (size_t i = 0; i < n; ++i) out[i] = lo + (hi - lo) * u01(orc_splitmix64_at(seed, i));
}

/* Normal(mean, std): Box-Muller on draws 2i, 2i+1; u1 in (0, 1]. */
void orc_fill_normal_f32(uint64_t seed, size_t n, float mean, float std, float* out) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i) {
        const double u1 = 1.0 - u01(orc_splitmix64_at(seed, 2 * i));
        const double u2 = u01(orc_splitmix64_at(seed, 2 * i + 1));
        out[i] = (float)(mean + std * sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

/* Integers uniform on [lo, hi] (inclusive). */
void orc_fill_int_i32(uint64_t seed, size_t n, int32_t lo, int32_t hi, int32_t* out) {
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; ++i) out[i] = (int32_t)((int64_t)lo + (int64_t)(orc_splitmix64_at(seed, i) % span));
}
void orc_fill_int_i64(uint64_t seed, size_t n, int64_t lo, int64_t hi, int64_t* out) {
    const uint64_t span = (uint64_t)(hi - lo) + 1u;
    for (size_t i = 0; i < n; ++i) out[i] = lo + (int64_t)(orc_splitmix64_at(seed, i) % span);
}

/* ---- fp16 / bf16 round-to-nearest-even -------------------------------------------------- */

static uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = fbits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* Result is subnormal (or zero): value in units of 2^-24 is m * 2^-(126 - exp). */
        const int shift = 126 - (int)exp;
        if (shift > 24) return (uint16_t)sign;
        const uint32_t m = mant | 0x800000u;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t v = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rb = mant & 0x1fffu;
    if (rb > 0x1000u || (rb == 0x1000u && (v & 1u))) ++v;   /* may carry into inf: correct */
    return (uint16_t)(sign | v);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t mant = (uint32_t)h & 0x3ffu;
    if (exp == 0) {
        const float v = (float)mant * (1.0f / 16777216.0f);   /* mant * 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return bitsf(sign | 0x7f800000u | (mant << 13));
    return bitsf(sign | ((exp + 112u) << 23) | (mant << 13));
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = fbits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return bitsf((uint32_t)b << 16); }

/* Round an fp32 array to f16 (kind 1) or bf16 (kind 2): rounded values and their bits. */
void orc_round(int kind, const float* in, size_t n, float* out_vals, uint16_t* out_bits) {
    for (size_t i = 0; i < n; ++i) {
        const uint16_t b = (kind == 2) ? orc_f32_to_bf16(in[i]) : orc_f32_to_f16(in[i]);
        if (out_bits) out_bits[i] = b;
        if (out_vals) out_vals[i] = (kind == 2) ? orc_bf16_to_f32(b) : orc_f16_to_f32(b);
    }
}

void orc_widen(int kind, const uint16_t* in, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (kind == 2) ? orc_bf16_to_f32(in[i]) : orc_f16_to_f32(in[i]);
}

/* ---- attention -------------------------------------------------------------------------- */

/* One query row; same operation order as cpu_prefill (validate_attention_api.hip:35-48). */
static void prefill_row(const float* qp, const float* Kh, const float* Vh, float* op, float* S, int D, int kmax,
                        float scale) {
    float mx = -1e38f;
    for (int k = 0; k < kmax; ++k) {
        float dot = 0;
        const float* kp = Kh + (size_t)k * D;
        for (int d = 0; d < D; ++d) dot += qp[d] * kp[d];
        S[k] = dot * scale;
        mx = S[k] > mx ? S[k] : mx;
    }
    float se = 0;
    for (int k = 0; k < kmax; ++k) { S[k] = expf(S[k] - mx); se += S[k]; }
    for (int k = 0; k < kmax; ++k) S[k] /= se;
    for (int d = 0; d < D; ++d) {
        float o = 0;
        for (int k = 0; k < kmax; ++k) o += S[k] * Vh[(size_t)k * D + d];
        op[d] = o;
    }
}

/* Q, O [batch][nQH][seqQ][D]; K, V [batch][nKVH][seqK][D]. Returns 0, or -1 on bad args. */
int orc_prefill_f32(const float* Q, const float* K, const float* V, float* O, int D, int seqQ, int seqK, int nQH,
                    int nKVH, int batch, int causal) {
    if (D <= 0 || seqQ <= 0 || seqK <= 0 || nQH <= 0 || nKVH <= 0 || batch <= 0 || nQH % nKVH) return -1;
    const float scale = 1.f / sqrtf((float)D);
    const int group = nQH / nKVH;
    float* S = (float*)malloc(sizeof(float) * (size_t)seqK);
    if (!S) return -1;
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < nQH; ++h) {
            const int kvh = h / group;
            const float* Kh = K + ((size_t)b * nKVH + kvh) * (size_t)seqK * D;
            const float* Vh = V + ((size_t)b * nKVH + kvh) * (size_t)seqK * D;
            for (int q = 0; q < seqQ; ++q) {
                const int kmax = causal ? (seqK < q + 1 ? seqK : q + 1) : seqK;
                prefill_row(Q + (((size_t)b * nQH + h) * seqQ + q) * D, Kh, Vh,
                            O + (((size_t)b * nQH + h) * seqQ + q) * D, S, D, kmax, scale);
            }
        }
    free(S);
    return 0;
}

/* Selected rows: rows[3*i..3*i+2] = (b, h, q); out is [nrows][D]. */
int orc_prefill_rows(const float* Q, const float* K, const float* V, int D, int seqQ, int seqK, int nQH, int nKVH,
                     int batch, int causal, const int32_t* rows, size_t nrows, float* out) {
    if (D <= 0 || seqQ <= 0 || seqK <= 0 || nQH <= 0 || nKVH <= 0 || batch <= 0 || nQH % nKVH) return -1;
    const float scale = 1.f / sqrtf((float)D);
    const int group = nQH / nKVH;
    float* S = (float*)malloc(sizeof(float) * (size_t)seqK);
    if (!S) return -1;
    for (size_t i = 0; i < nrows; ++i) {
        const int b = rows[3 * i], h = rows[3 * i + 1], q = rows[3 * i + 2];
        if (b < 0 || b >= batch || h < 0 || h >= nQH || q < 0 || q >= seqQ) { free(S); return -1; }
        const int kvh = h / group;
        const int kmax = causal ? (seqK < q + 1 ? seqK : q + 1) : seqK;
        prefill_row(Q + (((size_t)b * nQH + h) * seqQ + q) * D, K + ((size_t)b * nKVH + kvh) * (size_t)seqK * D,
                    V + ((size_t)b * nKVH + kvh) * (size_t)seqK * D, out + i * D, S, D, kmax, scale);
    }
    free(S);
    return 0;
}

/* q, o [batch][nQH][D]; K, V [batch][nKVH][stride][D] (stride 0 = N). Operation order of
 * cpu_decode (validate_attention_api.hip:58-70). */
int orc_decode_f32(const float* q, const float* K, const float* V, float* o, int D, int N, int nQH, int nKVH,
                   int batch, int stride) {
    if (D <= 0 || N <= 0 || nQH <= 0 || nKVH <= 0 || batch <= 0 || nQH % nKVH) return -1;
    if (stride == 0) stride = N;
    if (stride < N) return -1;
    const float scale = 1.f / sqrtf((float)D);
    const int group = nQH / nKVH;
    float* S = (float*)malloc(sizeof(float) * (size_t)N);
    if (!S) return -1;
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < nQH; ++h) {
            const int kvh = h / group;
            const float* Kh = K + ((size_t)b * nKVH + kvh) * (size_t)stride * D;
            const float* Vh = V + ((size_t)b * nKVH + kvh) * (size_t)stride * D;
            const float* qp = q + ((size_t)b * nQH + h) * D;
            float mx = -1e38f;
            for (int k = 0; k < N; ++k) {
                float dot = 0;
                const float* kp = Kh + (size_t)k * D;
                for (int d = 0; d < D; ++d) dot += qp[d] * kp[d];
                S[k] = dot * scale;
                mx = S[k] > mx ? S[k] : mx;
            }
            float se = 0;
            for (int k = 0; k < N; ++k) { S[k] = expf(S[k] - mx); se += S[k]; }
            float* op = o + ((size_t)b * nQH + h) * D;
            for (int d = 0; d < D; ++d) {
                float acc = 0;
                for (int k = 0; k < N; ++k) acc += (S[k] / se) * Vh[(size_t)k * D + d];
                op[d] = acc;
            }
        }
    free(S);
    return 0;
}

/* ---- reduce / scan ----------------------------------------------------------------------- *
 * dtype: 0 f32, 1 f16 bits, 2 bf16 bits, 3 f64, 4 i32, 5 i64 (the library's CDNA4_* codes).
 * op: 0 sum, 1 max, 2 min. Float inputs are combined in double and returned as double;
 * integer sums wrap in two's complement (the unsigned type), results in the input type.
 * n == 0 yields the operator's identity. */

static double load_f(int dtype, const void* in, size_t i) {
    switch (dtype) {
        case 0: return (double)((const float*)in)[i];
        case 1: return (double)orc_f16_to_f32(((const uint16_t*)in)[i]);
        case 2: return (double)orc_bf16_to_f32(((const uint16_t*)in)[i]);
        default: return ((const double*)in)[i];
    }
}

int orc_reduce(int op, int dtype, const void* in, size_t n, void* out) {
    if (op < 0 || op > 2 || dtype < 0 || dtype > 5) return -1;
    if (dtype == 4) {
        const int32_t* x = (const int32_t*)in;
        uint32_t s = 0; int32_t mx = INT32_MIN, mn = INT32_MAX;
        for (size_t i = 0; i < n; ++i) { s += (uint32_t)x[i]; if (x[i] > mx) mx = x[i]; if (x[i] < mn) mn = x[i]; }
        *(int32_t*)out = op == 0 ? (int32_t)s : (op == 1 ? mx : mn);
        return 0;
    }
    if (dtype == 5) {
        const int64_t* x = (const int64_t*)in;
        uint64_t s = 0; int64_t mx = INT64_MIN, mn = INT64_MAX;
        for (size_t i = 0; i < n; ++i) { s += (uint64_t)x[i]; if (x[i] > mx) mx = x[i]; if (x[i] < mn) mn = x[i]; }
        *(int64_t*)out = op == 0 ? (int64_t)s : (op == 1 ? mx : mn);
        return 0;
    }
    double s = 0.0, mx = -INFINITY, mn = INFINITY;
    for (size_t i = 0; i < n; ++i) {
        const double v = load_f(dtype, in, i);
        s += v; if (v > mx) mx = v; if (v < mn) mn = v;
    }
    if (dtype == 3) {   /* f64 identities are lowest / max of double */
        if (n == 0) { mx = -1.7976931348623157e308; mn = 1.7976931348623157e308; }
    } else if (n == 0) {
        mx = -3.4028234663852886e38; mn = 3.4028234663852886e38;   /* float lowest / max */
    }
    *(double*)out = op == 0 ? s : (op == 1 ? mx : mn);
    return 0;
}

int orc_scan_inclusive(int op, int dtype, const void* in, size_t n, void* out) {
    if (op < 0 || op > 2 || dtype < 0 || dtype > 5) return -1;
    if (dtype == 4) {
        const int32_t* x = (const int32_t*)in; int32_t* y = (int32_t*)out;
        uint32_t s = 0; int32_t a = 0;
        for (size_t i = 0; i < n; ++i) {
            if (op == 0) { s += (uint32_t)x[i]; y[i] = (int32_t)s; }
            else { a = (i == 0) ? x[i] : (op == 1 ? (x[i] > a ? x[i] : a) : (x[i] < a ? x[i] : a)); y[i] = a; }
        }
        return 0;
    }
    if (dtype == 5) {
        const int64_t* x = (const int64_t*)in; int64_t* y = (int64_t*)out;
        uint64_t s = 0; int64_t a = 0;
        for (size_t i = 0; i < n; ++i) {
            if (op == 0) { s += (uint64_t)x[i]; y[i] = (int64_t)s; }
            else { a = (i == 0) ? x[i] : (op == 1 ? (x[i] > a ? x[i] : a) : (x[i] < a ? x[i] : a)); y[i] = a; }
        }
        return 0;
    }
    double* y = (double*)out;
    double a = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double v = load_f(dtype, in, i);
        if (i == 0) a = v;
        else if (op == 0) a += v;
        else if (op == 1) a = v > a ? v : a;
        else a = v < a ? v : a;
        y[i] = a;
    }
    return 0;
}

/* ---- norms and RoPE ---------------------------------------------------------------------- */

/* forward.hpp:34-56 with the block reduction replaced by a sequential fp32 sum. */
void orc_rmsnorm_f32(const float* X, const uint16_t* W, float* Y, int M, int H, float eps) {
    for (int r = 0; r < M; ++r) {
        const float* x = X + (size_t)r * H;
        float* y = Y + (size_t)r * H;
        float ss = 0.f;
        for (int i = 0; i < H; ++i) ss += x[i] * x[i];
        const float inv = 1.0f / sqrtf(ss / (float)H + eps);
        for (int i = 0; i < H; ++i) y[i] = x[i] * inv * orc_f16_to_f32(W[i]);
    }
}

/* bench_layernorm.hip:51-114, two passes, statistics in double. */
void orc_layernorm_f32(const float* X, const float* G, const float* B, float* Y, int M, int H, float eps) {
    for (int r = 0; r < M; ++r) {
        const float* x = X + (size_t)r * H;
        float* y = Y + (size_t)r * H;
        double s = 0.0;
        for (int i = 0; i < H; ++i) s += x[i];
        const double mean = s / H;
        double q = 0.0;
        for (int i = 0; i < H; ++i) { const double d = x[i] - mean; q += d * d; }
        const double inv = 1.0 / sqrt(q / H + (double)eps);
        for (int i = 0; i < H; ++i) y[i] = (float)((x[i] - mean) * inv * G[i] + B[i]);
    }
}

/* bench_softmax.hip:59-105: m = max of the row, e = exp(x - m), y = e * (1 / sum(e)); the sum and
 * the exponentials in double, rounded to float at the end. */
void orc_softmax_rows_f32(const float* X, float* Y, int M, int H) {
    for (int r = 0; r < M; ++r) {
        const float* x = X + (size_t)r * H;
        float* y = Y + (size_t)r * H;
        float m = -INFINITY;
        for (int i = 0; i < H; ++i) m = x[i] > m ? x[i] : m;
        double s = 0.0;
        for (int i = 0; i < H; ++i) s += exp((double)x[i] - (double)m);
        for (int i = 0; i < H; ++i) y[i] = (float)(exp((double)x[i] - (double)m) / s);
    }
}

/* session.hpp:120-135: freq = theta^(-2d/D), entries d and d + D/2 share the angle. */
void orc_rope_table(float* cosv, float* sinv, int pos0, int T, int D, float theta) {
    for (int s = 0; s < T; ++s) {
        const int pos = pos0 + s;
        for (int d = 0; d < D / 2; ++d) {
            const float freq = 1.f / powf(theta, (2.f * d) / D);
            const float ang = pos * freq;
            cosv[(size_t)s * D + d] = cosf(ang); cosv[(size_t)s * D + d + D / 2] = cosf(ang);
            sinv[(size_t)s * D + d] = sinf(ang); sinv[(size_t)s * D + d + D / 2] = sinf(ang);
        }
    }
}

/* forward.hpp:135-148 on T fp16 bits [seq][heads][D]; cos/sin [seq][D]. */
void orc_rope_f16(uint16_t* T, const float* cosv, const float* sinv, int seq, int heads, int D) {
    float* row = (float*)malloc(sizeof(float) * (size_t)D);
    if (!row) return;
    for (int s = 0; s < seq; ++s)
        for (int h = 0; h < heads; ++h) {
            uint16_t* t = T + ((size_t)s * heads + h) * D;
            for (int d = 0; d < D; ++d) row[d] = orc_f16_to_f32(t[d]);
            for (int d = 0; d < D; ++d) {
                const float c = cosv[(size_t)s * D + d], sn = sinv[(size_t)s * D + d];
                const float tr = (d < D / 2) ? -row[d + D / 2] : row[d - D / 2];
                t[d] = orc_f32_to_f16(row[d] * c + tr * sn);
            }
        }
    free(row);
}

/* ---- KV cache and layouts ---------------------------------------------------------------- */

/* forward.hpp:209-220: cache[h][pos0 + s][d] = src[s][h][d], cache [heads][max_seq][D]. */
void orc_scatter_kv_f16(const uint16_t* src, uint16_t* cache, int T, int heads, int D, int pos0, int max_seq) {
    for (int s = 0; s < T; ++s)
        for (int h = 0; h < heads; ++h)
            for (int d = 0; d < D; ++d)
                cache[((size_t)h * max_seq + pos0 + s) * D + d] = src[((size_t)s * heads + h) * D + d];
}

/* forward.hpp:190-205: dir 0 token-major [seq][heads][D] -> head-major [heads][seq][D], dir 1 back. */
void orc_repack_f16(const uint16_t* src, uint16_t* dst, int seq, int heads, int D, int dir) {
    for (int s = 0; s < seq; ++s)
        for (int h = 0; h < heads; ++h)
            for (int d = 0; d < D; ++d) {
                const size_t tok = ((size_t)s * heads + h) * D + d;
                const size_t hm = ((size_t)h * seq + s) * D + d;
                if (dir == 0) dst[hm] = src[tok]; else dst[tok] = src[hm];
            }
}

/* session.hpp:170-199 in sequence: RoPE on copies of q and k (orc_rope_f16), q repacked to
 * head-major q_out, k and v scattered into the caches at pos0. */
void orc_rope_append_kv_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* q_out,
                            uint16_t* Kc, uint16_t* Vc, const float* cosv, const float* sinv, int T, int nQH,
                            int nKVH, int D, int pos0, int max_seq) {
    uint16_t* qr = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * nQH * D + 2);
    uint16_t* kr = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * nKVH * D + 2);
    if (!qr || !kr) { free(qr); free(kr); return; }
    memcpy(qr, q, sizeof(uint16_t) * (size_t)T * nQH * D);
    memcpy(kr, k, sizeof(uint16_t) * (size_t)T * nKVH * D);
    orc_rope_f16(qr, cosv, sinv, T, nQH, D);
    orc_rope_f16(kr, cosv, sinv, T, nKVH, D);
    orc_repack_f16(qr, q_out, T, nQH, D, 0);
    orc_scatter_kv_f16(kr, Kc, T, nKVH, D, pos0, max_seq);
    orc_scatter_kv_f16(v, Vc, T, nKVH, D, pos0, max_seq);
    free(qr);
    free(kr);
}
