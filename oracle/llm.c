/*
 * CPU oracle of the small-LLM runtime's layer loop. TEST INFRASTRUCTURE ONLY: called by tests/
 * as the checker and by bench.py's cpu_baseline leg, never by the product library.
 *
 * Restates, single-threaded in fp32 with the reference's rounding points:
 *   Session::run_layers   cdna3-prims/include/cdna3/runtime/session.hpp:141-238
 *     rmsnorm_f32_kernel  forward.hpp:34-56 (eps 1e-6), then the f32 -> f16 cast before each GEMM
 *                         (rocblas_gemm.hpp:36-41, :150-178)
 *     Q/K/V GEMM          f16 x f16, fp32 accumulate, f16 result (rocblas_gemm.hpp:150-178), then
 *                         bias_add_f16_kernel (rocblas_gemm.hpp:58-63): f16(f32(y) + f32(b))
 *     rope_kernel         forward.hpp:135-148 on Q and K, table of Session::fill_rope
 *                         (session.hpp:120-135)
 *     append_kv           session.hpp:240-250: K/V rows into the cache [L][nKV][max_seq][D]
 *     attention           causal softmax attention of each query over cache rows 0..pos, as
 *                         cpu_decode (cdna3-prims/tests/validate_attention_api.hip:53-72), output
 *                         rounded to f16 (the attention kernels write fp16)
 *     O-proj + residual   f16 x f16 -> f32 (rocblas_gemm.hpp:187-209), add_f32_kernel
 *     MLP                 gate/up f32 (:112-141), silu_mul_f32_kernel (forward.hpp:154-160), f16
 *                         cast, down f32, residual
 *     final norm          fp32 (session.hpp:233-236)
 *   greedy_from_last      session.hpp:320-331: logits = final-norm(hidden) . lm_head^T, fp32
 *                         accumulation from the fp32 normed row, stored as fp16
 *                         (gemm_f32in_f16out_kernel, forward.hpp:70-86); the argmax over them
 *                         (argmax_kernel, forward.hpp:244-262) is restated in oracle/__init__.py.
 * Extension (no reference counterpart): "layernorm" models use the two-pass LayerNorm of
 * research/wave-primitives/benchmarks/bench_layernorm.hip:51-114 (eps 1e-5) with f16 gamma/beta.
 * The embedding row is widened to fp32 (embed_gather_f32_kernel, forward.hpp:174-183).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_rope_table(float* cosv, float* sinv, int pos0, int T, int D, float theta);

/* Weights are fp32 arrays holding the model's fp16 values exactly; per-layer tensors are arrays
 * of n_layers pointers. Biases and norm betas may be NULL. */
typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, layernorm;
    float rope_theta, eps;
    const float *embed, *lm_head, *fnorm, *fnorm_b;
    const float *const *wq, *const *wk, *const *wv, *const *wo;
    const float *const *bq, *const *bk, *const *bv;
    const float *const *wg, *const *wu, *const *wd;
    const float *const *n1, *const *n1b, *const *n2, *const *n2b;
} orc_llm;

static float r16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

/* Dot product with eight running partial sums (fixed order; lets the compiler vectorise). */
static float dot(const float* a, const float* b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
    float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* y[r][n] = x[r] . W[n] for W [N][K]. */
static void matvec_rows(const float* x, int T, const float* W, int N, int K, float* y) {
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < N; ++n) y[(size_t)t * N + n] = dot(x + (size_t)t * K, W + (size_t)n * K, K);
}

static void norm_rows(const orc_llm* m, const float* X, const float* g, const float* b, float* Y, int T) {
    const int H = m->hidden;
    for (int t = 0; t < T; ++t) {
        const float* x = X + (size_t)t * H;
        float* y = Y + (size_t)t * H;
        if (m->layernorm) {
            double s = 0.0, q = 0.0;
            for (int i = 0; i < H; ++i) s += x[i];
            const double mean = s / H;
            for (int i = 0; i < H; ++i) { const double d = x[i] - mean; q += d * d; }
            const double inv = 1.0 / sqrt(q / H + (double)m->eps);
            for (int i = 0; i < H; ++i) y[i] = (float)((x[i] - mean) * inv * g[i] + (b ? b[i] : 0.f));
        } else {
            float ss = 0.f;
            for (int i = 0; i < H; ++i) ss += x[i] * x[i];
            const float inv = 1.0f / sqrtf(ss / (float)H + m->eps);
            for (int i = 0; i < H; ++i) y[i] = x[i] * inv * g[i] + (b ? b[i] : 0.f);
        }
    }
}

/* Rotate-half RoPE of one head row (f16 values in, f16-rounded out). */
static void rope_row(float* t, const float* c, const float* s, int D, float* tmp) {
    memcpy(tmp, t, sizeof(float) * (size_t)D);
    for (int d = 0; d < D; ++d) {
        const float tr = d < D / 2 ? -tmp[d + D / 2] : tmp[d - D / 2];
        t[d] = r16(tmp[d] * c[d] + tr * s[d]);
    }
}

/*
 * Runs T tokens (ids) at positions pos0 .. pos0+T-1 through every layer, appending their K/V to
 * the caches (fp16 bits [n_layers][n_kv_heads][max_seq][head_dim], rows < pos0 already filled),
 * and writes fp32 logits: [T][vocab] when all_logits, else [vocab] of the last token.
 * Returns 0, or -1 on bad arguments / allocation failure.
 */
int orc_llm_forward(const orc_llm* m, const int* ids, int T, int pos0, uint16_t* Kc, uint16_t* Vc, int max_seq,
                    float* logits, int all_logits) {
    const int L = m->n_layers, H = m->hidden, nH = m->n_heads, nKV = m->n_kv_heads, D = m->head_dim;
    const int F = m->ffn_dim, V = m->vocab, QD = nH * D, KVD = nKV * D;
    if (T < 1 || pos0 < 0 || pos0 + T > max_seq || nH % nKV || D % 2) return -1;
    for (int t = 0; t < T; ++t)
        if (ids[t] < 0 || ids[t] >= V) return -1;
    const int maxw = (QD > F ? QD : F) > H ? (QD > F ? QD : F) : H;
    float *h = malloc(sizeof(float) * (size_t)T * H), *xn = malloc(sizeof(float) * (size_t)T * maxw);
    float *q = malloc(sizeof(float) * (size_t)T * QD), *k = malloc(sizeof(float) * (size_t)T * KVD);
    float *v = malloc(sizeof(float) * (size_t)T * KVD), *att = malloc(sizeof(float) * (size_t)T * QD);
    float *g = malloc(sizeof(float) * (size_t)T * F), *u = malloc(sizeof(float) * (size_t)T * F);
    float *y = malloc(sizeof(float) * (size_t)T * (H > F ? H : F));
    float *cs = malloc(sizeof(float) * (size_t)T * D), *sn = malloc(sizeof(float) * (size_t)T * D);
    float *S = malloc(sizeof(float) * (size_t)(pos0 + T)), *tmp = malloc(sizeof(float) * (size_t)D);
    float *kr = malloc(sizeof(float) * (size_t)D);
    int rc = 0;
    if (!h || !xn || !q || !k || !v || !att || !g || !u || !y || !cs || !sn || !S || !tmp || !kr) {
        rc = -1;
        goto out;
    }
    orc_rope_table(cs, sn, pos0, T, D, m->rope_theta);
    for (int t = 0; t < T; ++t)
        memcpy(h + (size_t)t * H, m->embed + (size_t)ids[t] * H, sizeof(float) * (size_t)H);
    const float scale = 1.f / sqrtf((float)D);
    for (int l = 0; l < L; ++l) {
        uint16_t* Kl = Kc + (size_t)l * nKV * max_seq * D;
        uint16_t* Vl = Vc + (size_t)l * nKV * max_seq * D;
        norm_rows(m, h, m->n1[l], m->n1b ? m->n1b[l] : NULL, xn, T);
        for (size_t i = 0; i < (size_t)T * H; ++i) xn[i] = r16(xn[i]);
        matvec_rows(xn, T, m->wq[l], QD, H, q);
        matvec_rows(xn, T, m->wk[l], KVD, H, k);
        matvec_rows(xn, T, m->wv[l], KVD, H, v);
        for (int t = 0; t < T; ++t) {
            for (int i = 0; i < QD; ++i) {
                float* p = q + (size_t)t * QD + i;
                *p = r16(*p);
                if (m->bq && m->bq[l]) *p = r16(*p + m->bq[l][i]);
            }
            for (int i = 0; i < KVD; ++i) {
                float *pk = k + (size_t)t * KVD + i, *pv = v + (size_t)t * KVD + i;
                *pk = r16(*pk);
                *pv = r16(*pv);
                if (m->bk && m->bk[l]) *pk = r16(*pk + m->bk[l][i]);
                if (m->bv && m->bv[l]) *pv = r16(*pv + m->bv[l][i]);
            }
            for (int hh = 0; hh < nH; ++hh) rope_row(q + (size_t)t * QD + hh * D, cs + (size_t)t * D, sn + (size_t)t * D, D, tmp);
            for (int hh = 0; hh < nKV; ++hh) {
                rope_row(k + (size_t)t * KVD + hh * D, cs + (size_t)t * D, sn + (size_t)t * D, D, tmp);
                for (int d = 0; d < D; ++d) {
                    const size_t at = ((size_t)hh * max_seq + pos0 + t) * D + d;
                    Kl[at] = orc_f32_to_f16(k[(size_t)t * KVD + hh * D + d]);
                    Vl[at] = orc_f32_to_f16(v[(size_t)t * KVD + hh * D + d]);
                }
            }
        }
        /* causal attention of token t over cache rows 0 .. pos0 + t */
        for (int t = 0; t < T; ++t) {
            const int n = pos0 + t + 1;
            for (int hh = 0; hh < nH; ++hh) {
                const int kvh = hh / (nH / nKV);
                const float* qp = q + (size_t)t * QD + hh * D;
                float mx = -1e38f;
                for (int j = 0; j < n; ++j) {
                    const uint16_t* kp = Kl + ((size_t)kvh * max_seq + j) * D;
                    for (int d = 0; d < D; ++d) kr[d] = orc_f16_to_f32(kp[d]);
                    S[j] = dot(qp, kr, D) * scale;
                    mx = S[j] > mx ? S[j] : mx;
                }
                float l_sum = 0.f;
                for (int j = 0; j < n; ++j) {
                    S[j] = expf(S[j] - mx);
                    l_sum += S[j];
                }
                float* o = att + (size_t)t * QD + hh * D;
                for (int d = 0; d < D; ++d) o[d] = 0.f;
                for (int j = 0; j < n; ++j) {
                    const uint16_t* vp = Vl + ((size_t)kvh * max_seq + j) * D;
                    for (int d = 0; d < D; ++d) o[d] += S[j] * orc_f16_to_f32(vp[d]);
                }
                for (int d = 0; d < D; ++d) o[d] = r16(o[d] / l_sum);
            }
        }
        matvec_rows(att, T, m->wo[l], H, QD, y);
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] += y[i];
        norm_rows(m, h, m->n2[l], m->n2b ? m->n2b[l] : NULL, xn, T);
        for (size_t i = 0; i < (size_t)T * H; ++i) xn[i] = r16(xn[i]);
        matvec_rows(xn, T, m->wg[l], F, H, g);
        matvec_rows(xn, T, m->wu[l], F, H, u);
        for (size_t i = 0; i < (size_t)T * F; ++i) g[i] = r16((g[i] / (1.f + expf(-g[i]))) * u[i]);
        matvec_rows(g, T, m->wd[l], H, F, y);
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] += y[i];
    }
    {
        const int t0 = all_logits ? 0 : T - 1;
        const int nt = T - t0;
        norm_rows(m, h + (size_t)t0 * H, m->fnorm, m->fnorm_b, xn, nt);
        matvec_rows(xn, nt, m->lm_head, V, H, logits);
        for (size_t i = 0; i < (size_t)nt * V; ++i) logits[i] = r16(logits[i]);   /* the fp16 logits store */
    }
out:
    free(h); free(xn); free(q); free(k); free(v); free(att); free(g); free(u); free(y);
    free(cs); free(sn); free(S); free(tmp); free(kr);
    return rc;
}
