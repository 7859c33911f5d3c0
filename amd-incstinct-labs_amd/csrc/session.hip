// Greedy batch-1 LLM session for gfx950: model loading and the layer loop of the reference's
// runtime, on the library's own kernels.
//
// Reference behaviour restated (cdna3-prims/include/cdna3/runtime/): ModelLoader (model_loader.hpp:
// 130-193, meta.json + one raw fp16 .bin per tensor), Session::run_layers (session.hpp:141-235:
// norm, Q/K/V projections + bias, RoPE, KV append, causal prefill or strided decode, O projection
// + residual, norm, SiLU-gated MLP + residual, final norm) and Session::generate / greedy_from_last
// (session.hpp:262-338: prefill the prompt, then one token at a time, lm_head + argmax).
//
// MI355X design (host C++ over the library's kernels, one HIP stream per session):
//   * Weights are loaded once; Q/K/V rows are concatenated into one matrix (and their biases into
//     one vector), gate and up rows into one, so the decode step reads each as a single stream.
//   * Prompt (T > 1): the projections are the library's MFMA GEMMs (f16 in, f32 accumulate; the O
//     and down projections accumulate into the fp32 residual, the gate|up GEMM writes the SiLU
//     product; rocBLAS for shapes they do not take), RoPE + KV append is one fused
//     launch that also writes Q head-major, and the causal prefill reads K/V in place from the
//     cache and writes O token-major for the O projection (no repacks).
//   * Decode (T = 1): every projection is an HBM-streaming GEMV with its epilogue fused (bias,
//     residual add, SiLU product); attention is the decode over the strided cache, for short
//     caches as a few split-K partials per head that the O projection's GEMV merges as it loads
//     its input vector.
//   * The RoPE table for every position is built once on the device. The next token id never
//     leaves the device: argmax writes it, and the token's embedding row as the next step's
//     input, so a generation of N tokens is one queue of launches and one copy back at the end
//     (unless an EOS id must be checked after each step).
//   * The decode step is captured once as a HIP graph and replayed: the position and the token
//     index live in a device step state that the kernels read and the argmax advances, so one
//     graph serves every step with the same attention plan (re-captured when the plan changes
//     with the cache length). CDNA4_SESSION_GRAPH=0 launches the same kernels one by one.
//   * The prompt's GEMMs run on the library's own MFMA GEMM (gemm.hip) when their shapes
//     allow, otherwise on rocBLAS; CDNA4_SESSION_ROCBLAS=1 sends all to rocBLAS.
#include "common.hpp"
#include <rocblas/rocblas.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>
#include <exception>
#include <map>
#include <string>
#include <vector>

namespace cdna4 {

int llm_embed(const void* embed, const int* ids, float* out, int T, int H, int V, hipStream_t s);
int llm_norm_cast(bool layer, const float* X, const void* W, const void* B, void* Y, int M, int H, float eps,
                  hipStream_t s);
int llm_gemv_residual(const void* x, const void* W, float* out, int N, int K, hipStream_t s);
int llm_gemv_qkv(bool layer, const float* hidden, const void* gain, const void* beta, float eps, const void* W,
                 const void* bias, int H, int D, int nH, int nKV, const float* cos_row, const float* sin_row,
                 void* q_out, void* Kc, void* Vc, int pos, int max_seq, hipStream_t s,
                 const int* pos_dev = nullptr);
int llm_gemv_silu(bool layer, const float* hidden, const void* gain, const void* beta, float eps, const void* W,
                  void* act, int F, int H, hipStream_t s);
size_t llm_argmax_partials(int V);
int llm_logits_argmax(bool layer, const float* hidden, const void* gain, const void* beta, float eps,
                      const void* W, float* logits, int V, int H, unsigned long long* partial,
                      unsigned long long* scratch16, int* ids, int* tokens, int step, hipStream_t s,
                      int* state = nullptr, const void* embed = nullptr, float* next_row = nullptr);
int llm_step_state(int* state, int pos, int step, hipStream_t s);
long long attn_decode_plan_key(const cdna3_decode_cfg& c);
int attn_decode_replayable(const void* q, const void* K, const void* V, void* o, const cdna3_decode_cfg& c, int dtype,
                           void* ws, size_t ws_bytes, const int* len_pos, hipStream_t s);
int llm_silu_mul(const float* gu, void* act, int T, int F, hipStream_t s);
int llm_gemv_residual_merge(const float* part_ml, const float* part_o, int P, int D, const void* W, float* out, int N,
                            int K, hipStream_t s);
size_t attn_decode_partials_bytes(const cdna3_decode_cfg& c, int P);
int attn_decode_partials(const void* q, const void* K, const void* V, const cdna3_decode_cfg& c, int dtype, int P,
                         void* ws, size_t ws_bytes, const int* len_pos, hipStream_t s);
int llm_gemm_f16(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, bool accum, int M, int N, int K, int ldy,
                 hipStream_t s, bool cold);
int llm_gemm_qkv_rope(const uint16_t* X, const uint16_t* W, int M, int K, const QkvOut& qe, hipStream_t s);
int llm_gemm_f16_silu(const uint16_t* X, const uint16_t* W, void* Y, int M, int F, int K, int ldy, hipStream_t s);
int llm_bias_add_f16(void* Y, const void* b, int T, int N, hipStream_t s);
int kv_rope_append(const void* q, const void* k, const void* v, long long ldq, long long ldk, long long ldv,
                   void* q_out, void* K_cache, void* V_cache, const float* cos_tab, const float* sin_tab, int T,
                   int nQH, int nKVH, int D, int pos0, int max_seq, hipStream_t stream);

namespace {

#define CK(expr)                                   \
    do {                                           \
        const int e_ = (int)(expr);                \
        if (e_ != 0) return e_;                    \
    } while (0)

// meta.json of the reference's exporter: one flat object of "key": value pairs.
bool parse_meta(const std::string& path, std::map<std::string, std::string>& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    std::string s;
    char buf[4096];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    fclose(f);
    size_t i = 0;
    auto skip = [&] { while (i < s.size() && strchr(" \t\r\n,{}", s[i])) ++i; };
    while (true) {
        skip();
        if (i >= s.size() || s[i] != '"') break;
        const size_t k0 = ++i;
        while (i < s.size() && s[i] != '"') ++i;
        const std::string key = s.substr(k0, i - k0);
        ++i;
        while (i < s.size() && (s[i] == ' ' || s[i] == ':')) ++i;
        std::string val;
        if (i < s.size() && s[i] == '"') {
            const size_t v0 = ++i;
            while (i < s.size() && s[i] != '"') ++i;
            val = s.substr(v0, i - v0);
            ++i;
        } else {
            const size_t v0 = i;
            while (i < s.size() && !strchr(",}\r\n", s[i])) ++i;
            val = s.substr(v0, i - v0);
            while (!val.empty() && val.back() == ' ') val.pop_back();
        }
        out[key] = val;
    }
    return true;
}

// Appends the raw fp16 tensor at path (exactly `count` elements) to host.
bool read_f16(const std::string& path, size_t count, std::vector<uint16_t>& host) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    const size_t at = host.size();
    host.resize(at + count);
    const size_t got = fread(host.data() + at, 2, count, f);
    char extra;
    const bool more = fread(&extra, 1, 1, f) == 1;
    fclose(f);
    return got == count && !more;
}

struct Layer {
    uint16_t *wqkv = nullptr, *bqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wdown = nullptr;
    uint16_t *n_attn = nullptr, *n_attn_b = nullptr, *n_mlp = nullptr, *n_mlp_b = nullptr;
};

}  // namespace

struct Session {
    cdna3_model_cfg c{};
    int max_seq = 0;
    std::vector<Layer> L;
    uint16_t *embed = nullptr, *lm_head = nullptr, *fnorm = nullptr, *fnorm_b = nullptr;
    uint16_t *Kc = nullptr, *Vc = nullptr;            // [layers][nKVH][max_seq][D]
    float *cos_tab = nullptr, *sin_tab = nullptr;     // [max_seq][D]
    void* dec_ws = nullptr;
    size_t dec_ws_bytes = 0;
    rocblas_handle blas = nullptr;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    // scratch, sized for `cap` tokens
    int cap = 0;
    float *hidden = nullptr, *gu = nullptr, *logits = nullptr;
    unsigned long long *partial = nullptr, *scratch16 = nullptr;
    uint16_t *xn = nullptr, *q = nullptr, *qh = nullptr, *attn = nullptr, *act = nullptr;   // q: [T][QD + 2 KVD]
    int *ids = nullptr, *tokens = nullptr;
    std::vector<void*> scratch;
    // Captured decode step: one graph replayed for every step whose attention plan matches gkey;
    // positions and the token index live in the device step state dstate = {pos, step}.
    int* dstate = nullptr;
    bool use_graph = true;
    bool rocblas_only = false;   // CDNA4_SESSION_ROCBLAS=1: prompt GEMMs through rocBLAS only
    bool qkv_fused = true;       // CDNA4_SESSION_QKV_FUSED=0: prompt Q|K|V GEMM, then the separate append
    // Decode steps over a short cache (the one-launch attention plan): the attention runs as
    // attn_parts split-K partials per head, merged by the O-projection GEMV (0: the one-launch
    // attention and a plain GEMV). CDNA4_SESSION_ATTN_PARTS overrides it (0 .. 4). At config 5
    // (12 heads, 512-640 keys) 3 measured 269.4 us per token against 274.3 for 0, 269.7 for 2
    // and 271.3 for 4: the attention kernel drops from 6.5 to 4.9 us per layer.
    int attn_parts = 3;
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    long long gkey = -1;

    int dmalloc(void** p, size_t bytes, bool is_scratch = false) {
        CK(hipMalloc(p, bytes ? bytes : 16));
        (is_scratch ? scratch : allocs).push_back(*p);
        return 0;
    }
    int upload(uint16_t** dst, const std::vector<uint16_t>& host) {
        CK(dmalloc((void**)dst, host.size() * 2));
        CK(hipMemcpy(*dst, host.data(), host.size() * 2, hipMemcpyHostToDevice));
        return 0;
    }
    int qd() const { return c.n_heads * c.head_dim; }
    int kvd() const { return c.n_kv_heads * c.head_dim; }
    size_t layer_kv() const { return (size_t)c.n_kv_heads * max_seq * c.head_dim; }

    int read_config(const std::string& dir);
    int load(const std::string& dir);
    int reserve(int T);
    int gemm(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, float beta, int M, int N, int K, int ldy);
    int run_layers(int T, int pos0, const int* pos_dev = nullptr);
    int prefill(const int* host_ids, int T);
    int decode_step(int pos, int step, bool dev);
    int replay_step(int pos);
    void drop_graph() {
        if (gexec) (void)hipGraphExecDestroy(gexec);
        if (graph) (void)hipGraphDestroy(graph);
        gexec = nullptr;
        graph = nullptr;
        gkey = -1;
    }
    int check_ids(const int* host_ids, int T) const {
        if (T < 1 || T > max_seq) return CDNA4_ERR_INVALID_VALUE;
        for (int i = 0; i < T; ++i)
            if (host_ids[i] < 0 || host_ids[i] >= c.vocab_size) return CDNA4_ERR_INVALID_VALUE;
        return 0;
    }
    int last_token_logits(int T, int step, int* state = nullptr);
    void release();
};

// meta.json -> c, validated; host only (runs before any device call).
int Session::read_config(const std::string& dir) {
    std::map<std::string, std::string> meta;
    if (!parse_meta(dir + "/meta.json", meta)) return CDNA4_ERR_INVALID_VALUE;
    auto geti = [&](const char* k, int def) { return meta.count(k) ? atoi(meta[k].c_str()) : def; };
    c.n_layers = geti("n_layers", 0);
    c.hidden = geti("hidden", 0);
    c.n_heads = geti("n_heads", 0);
    c.n_kv_heads = geti("n_kv_heads", c.n_heads);
    c.head_dim = geti("head_dim", c.n_heads ? c.hidden / c.n_heads : 0);
    c.ffn_dim = geti("ffn_dim", 0);
    c.vocab_size = geti("vocab_size", 0);
    c.rope_theta = meta.count("rope_theta") ? (float)atof(meta["rope_theta"].c_str()) : 10000.f;
    c.qkv_bias = meta.count("qkv_bias") && (meta["qkv_bias"] == "1" || meta["qkv_bias"] == "true");
    c.layernorm = meta.count("norm") && meta["norm"] == "layernorm";
    c.norm_eps = meta.count("norm_eps") ? (float)atof(meta["norm_eps"].c_str()) : (c.layernorm ? 1e-5f : 1e-6f);
    const int H = c.hidden, F = c.ffn_dim, V = c.vocab_size, D = c.head_dim;
    if (c.n_layers < 1 || H < 8 || H % 8 || H > 4096 || c.n_heads < 1 || c.n_kv_heads < 1 ||
        c.n_heads % c.n_kv_heads || (D != 64 && D != 128) || F < 8 || F % 8 || F > 8192 || V < 1 || !(c.rope_theta > 0.f) ||
        !(c.norm_eps >= 0.f))
        return CDNA4_ERR_INVALID_VALUE;
    return 0;
}

// Weights (Q|K|V and gate|up concatenated), KV cache, RoPE table, workspaces, rocBLAS handle.
int Session::load(const std::string& dir) {
    const int H = c.hidden, F = c.ffn_dim, V = c.vocab_size, D = c.head_dim;
    auto p = [&](const std::string& name) { return dir + "/" + name + ".bin"; };
    std::vector<uint16_t> h;
    auto one = [&](const std::string& name, size_t count, uint16_t** dst) -> int {
        h.clear();
        if (!read_f16(p(name), count, h)) return CDNA4_ERR_INVALID_VALUE;
        return upload(dst, h);
    };
    auto optional = [&](const std::string& name, size_t count, uint16_t** dst) -> int {
        FILE* f = fopen(p(name).c_str(), "rb");
        if (!f) return 0;
        fclose(f);
        return one(name, count, dst);
    };
    CK(one("embed_tokens", (size_t)V * H, &embed));
    CK(one("lm_head", (size_t)V * H, &lm_head));
    CK(one("final_norm", H, &fnorm));
    CK(optional("final_norm_bias", H, &fnorm_b));
    L.resize(c.n_layers);
    for (int i = 0; i < c.n_layers; ++i) {
        const std::string lp = "layer_" + std::to_string(i) + "_";
        Layer& l = L[i];
        h.clear();
        if (!read_f16(p(lp + "q_proj"), (size_t)qd() * H, h) || !read_f16(p(lp + "k_proj"), (size_t)kvd() * H, h) ||
            !read_f16(p(lp + "v_proj"), (size_t)kvd() * H, h))
            return CDNA4_ERR_INVALID_VALUE;
        CK(upload(&l.wqkv, h));
        if (c.qkv_bias) {
            h.clear();
            if (!read_f16(p(lp + "q_bias"), qd(), h) || !read_f16(p(lp + "k_bias"), kvd(), h) ||
                !read_f16(p(lp + "v_bias"), kvd(), h))
                return CDNA4_ERR_INVALID_VALUE;
            CK(upload(&l.bqkv, h));
        }
        CK(one(lp + "o_proj", (size_t)H * qd(), &l.wo));
        h.clear();
        if (!read_f16(p(lp + "gate_proj"), (size_t)F * H, h) || !read_f16(p(lp + "up_proj"), (size_t)F * H, h))
            return CDNA4_ERR_INVALID_VALUE;
        CK(upload(&l.wgu, h));
        CK(one(lp + "down_proj", (size_t)H * F, &l.wdown));
        CK(one(lp + "norm_attn", H, &l.n_attn));
        CK(one(lp + "norm_mlp", H, &l.n_mlp));
        CK(optional(lp + "norm_attn_bias", H, &l.n_attn_b));
        CK(optional(lp + "norm_mlp_bias", H, &l.n_mlp_b));
    }
    // KV cache, RoPE table for every position, decode workspace for any length up to max_seq.
    CK(dmalloc((void**)&Kc, layer_kv() * c.n_layers * 2));
    CK(dmalloc((void**)&Vc, layer_kv() * c.n_layers * 2));
    CK(dmalloc((void**)&cos_tab, (size_t)max_seq * D * 4));
    CK(dmalloc((void**)&sin_tab, (size_t)max_seq * D * 4));
    CK(cdna3_rope_table_f32(cos_tab, sin_tab, 0, max_seq, D, c.rope_theta, (cdna4_stream_t)stream));
    for (int n = 1; n <= max_seq; ++n) {   // the split count is not monotonic in n: take the max
        cdna3_decode_cfg dc{D, n, c.n_heads, c.n_kv_heads, 1, max_seq};
        const size_t b = cdna3_attn_decode_workspace_size(&dc);
        if (b > dec_ws_bytes) dec_ws_bytes = b;
    }
    if (attn_parts > 0) {
        cdna3_decode_cfg dc{D, max_seq, c.n_heads, c.n_kv_heads, 1, max_seq};
        dec_ws_bytes = std::max(dec_ws_bytes, attn_decode_partials_bytes(dc, attn_parts));
    }
    CK(dmalloc(&dec_ws, dec_ws_bytes));
    CK(dmalloc((void**)&logits, (size_t)V * 4));
    CK(dmalloc((void**)&partial, llm_argmax_partials(V) * 8));
    CK(dmalloc((void**)&scratch16, 16 * 8));
    CK(dmalloc((void**)&dstate, 2 * sizeof(int)));
    if (rocblas_create_handle(&blas) != rocblas_status_success) return CDNA4_ERR_INVALID_VALUE;
    if (rocblas_set_stream(blas, stream) != rocblas_status_success) return CDNA4_ERR_INVALID_VALUE;
    return (int)hipStreamSynchronize(stream);
}

int Session::reserve(int T) {
    if (T <= cap) return 0;
    drop_graph();   // it holds the old scratch addresses
    for (void* ptr : scratch) (void)hipFree(ptr);
    scratch.clear();
    const size_t H = c.hidden, F = c.ffn_dim;
    CK(dmalloc((void**)&hidden, T * H * 4, true));
    CK(dmalloc((void**)&gu, T * 2 * F * 4, true));
    CK(dmalloc((void**)&xn, T * (H > F ? H : F) * 2, true));
    CK(dmalloc((void**)&q, (size_t)T * (qd() + 2 * kvd()) * 2, true));
    CK(dmalloc((void**)&qh, (size_t)T * qd() * 2, true));
    CK(dmalloc((void**)&attn, (size_t)T * qd() * 2, true));
    CK(dmalloc((void**)&act, T * F * 2, true));
    CK(dmalloc((void**)&ids, (size_t)T * 4, true));
    CK(dmalloc((void**)&tokens, (size_t)(max_seq + 1) * 4, true));
    cap = T;
    return 0;
}

// Row-major Y[M][N] (leading dimension ldy) = X[M][K] W[N][K]^T + beta Y, fp16 X and W, fp32
// accumulation, fp32 or fp16 Y. rocBLAS is column-major: row-major Y is column-major Y^T [N][M],
// and Y^T = W X^T, where the row-major W [N][K] read column-major is W^T (so op(A) = transpose,
// lda = K) and the row-major X [M][K] read column-major is X^T (op(B) = none, ldb = K). The
// reference derives the same call (rocblas_gemm.hpp:8-20). The library's MFMA GEMM (gemm.hip)
// takes every product whose shape it allows, told that its operands arrive cold (from HBM or the
// Infinity Cache: the residual projections then take 64 x 32 tiles); at the cfg5 prompt (T 512,
// under the kernel trace) it measured Q|K|V 8.3 us, O ~5, gate|up 12.4, down 13.7 against
// rocBLAS's 16.8, 10.5, 14.8 and 16.5. rocBLAS serves the rest (and everything with
// CDNA4_SESSION_ROCBLAS=1).
int Session::gemm(const uint16_t* X, const uint16_t* W, void* Y, bool y_f32, float beta, int M, int N, int K,
                  int ldy) {
    if (!rocblas_only && (beta == 0.f || beta == 1.f)) {
        const int e = llm_gemm_f16(X, W, Y, y_f32, beta == 1.f, M, N, K, ldy, stream, true);   // cold operands
        if (e != -1) return e;   // -1: a shape the kernel does not take
    }
    const float alpha = 1.f;
    const rocblas_datatype yt = y_f32 ? rocblas_datatype_f32_r : rocblas_datatype_f16_r;
    const rocblas_status st = rocblas_gemm_ex(blas, rocblas_operation_transpose, rocblas_operation_none, N, M, K,
                                              &alpha, W, rocblas_datatype_f16_r, K, X, rocblas_datatype_f16_r, K,
                                              &beta, Y, yt, ldy, Y, yt, ldy, rocblas_datatype_f32_r,
                                              rocblas_gemm_algo_standard, 0, 0);
    return st == rocblas_status_success ? 0 : CDNA4_ERR_INVALID_VALUE;
}

int Session::run_layers(int T, int pos0, const int* pos_dev) {
    const int H = c.hidden, F = c.ffn_dim, D = c.head_dim, nH = c.n_heads, nKV = c.n_kv_heads;
    const int QD = qd(), KVD = kvd();
    const bool lnorm = c.layernorm != 0;
    const float eps = c.norm_eps;
    const cdna4_stream_t s = (cdna4_stream_t)stream;
    for (int li = 0; li < c.n_layers; ++li) {
        const Layer& l = L[li];
        uint16_t* Kl = Kc + layer_kv() * li;
        uint16_t* Vl = Vc + layer_kv() * li;
        if (T == 1) {
            // decode step: five launches and the attention; every GEMV streams its weights once
            const size_t rope_off = pos_dev ? 0 : (size_t)pos0 * D;   // replayed: the kernel adds pos * D
            CK(llm_gemv_qkv(lnorm, hidden, l.n_attn, l.n_attn_b, eps, l.wqkv, l.bqkv, H, D, nH, nKV,
                            cos_tab + rope_off, sin_tab + rope_off, qh, Kl, Vl, pos0, max_seq, stream, pos_dev));
            cdna3_decode_cfg dc{D, pos0 + 1, nH, nKV, 1, max_seq};
            const long long key = attn_decode_plan_key(dc);
            if (attn_parts > 0 && (key == 1 || key == 3)) {   // short cache: partials merged in the O GEMV
                CK(attn_decode_partials(qh, Kl, Vl, dc, CDNA4_F16, attn_parts, dec_ws, dec_ws_bytes, pos_dev,
                                        stream));
                const float* pml = (const float*)dec_ws;
                const float* po = (const float*)((const char*)dec_ws +
                                                 (((size_t)nH * attn_parts * 2 * sizeof(float) + 255) & ~(size_t)255));
                CK(llm_gemv_residual_merge(pml, po, attn_parts, D, l.wo, hidden, H, QD, stream));
            } else {
                if (pos_dev)
                    CK(attn_decode_replayable(qh, Kl, Vl, attn, dc, CDNA4_F16, dec_ws, dec_ws_bytes, pos_dev,
                                              stream));
                else
                    CK(cdna3_attn_decode(qh, Kl, Vl, attn, &dc, CDNA4_F16, dec_ws, dec_ws_bytes, s));
                CK(llm_gemv_residual(attn, l.wo, hidden, H, QD, stream));
            }
            CK(llm_gemv_silu(lnorm, hidden, l.n_mlp, l.n_mlp_b, eps, l.wgu, act, F, H, stream));
            CK(llm_gemv_residual(act, l.wdown, hidden, H, F, stream));
            continue;
        }
        CK(llm_norm_cast(lnorm, hidden, l.n_attn, l.n_attn_b, xn, T, H, eps, stream));
        // one GEMM for Q|K|V: row t of q is [q_t | k_t | v_t], QKVD = QD + 2 KVD wide. Without a
        // bias, the GEMM's epilogue rotates Q and K and writes Q head-major and K/V into the cache
        // (the separate append below rounds and rotates alike).
        const int QKVD = QD + 2 * KVD;
        int qkv = -1;
        if (!l.bqkv && !rocblas_only && qkv_fused) {
            const QkvOut qe{qh, Kl, Vl, cos_tab, sin_tab, QD, KVD, D, T, pos0, max_seq};
            qkv = llm_gemm_qkv_rope(xn, l.wqkv, T, H, qe, stream);
        }
        if (qkv == -1) {
            CK(gemm(xn, l.wqkv, q, false, 0.f, T, QKVD, H, QKVD));
            if (l.bqkv) CK(llm_bias_add_f16(q, l.bqkv, T, QKVD, stream));
            CK(kv_rope_append(q, q + QD, q + QD + KVD, QKVD, QKVD, QKVD, qh, Kl, Vl, cos_tab + (size_t)pos0 * D,
                              sin_tab + (size_t)pos0 * D, T, nH, nKV, D, pos0, max_seq, stream));
        } else {
            CK(qkv);
        }
        // Prompt from an empty cache (pos0 == 0): causal over the T cached keys, read in place;
        // O written token-major for the O projection.
        cdna3_prefill_cfg pc{D, T, T, nH, nKV, 1, 1};
        cdna3_prefill_strides ps;
        ps.q_row = D; ps.q_head = (long long)T * D; ps.q_batch = ps.q_head * nH;
        ps.kv_row = D; ps.kv_head = (long long)max_seq * D; ps.kv_batch = ps.kv_head * nKV;
        ps.o_row = QD; ps.o_head = D; ps.o_batch = (long long)T * QD;
        CK(cdna3_attn_prefill_strided(qh, Kl, Vl, attn, &pc, &ps, CDNA4_F16, s));
        CK(gemm(attn, l.wo, hidden, true, 1.f, T, H, QD, H));
        CK(llm_norm_cast(lnorm, hidden, l.n_mlp, l.n_mlp_b, xn, T, H, eps, stream));
        // gate|up and the SiLU product in one launch where the library GEMM takes the shape
        const int fused = rocblas_only ? -1 : llm_gemm_f16_silu(xn, l.wgu, act, T, F, H, F, stream);
        if (fused == -1) {
            CK(gemm(xn, l.wgu, gu, true, 0.f, T, 2 * F, H, 2 * F));
            CK(llm_silu_mul(gu, act, T, F, stream));
        } else {
            CK(fused);
        }
        CK(gemm(act, l.wdown, hidden, true, 1.f, T, H, F, H));
    }
    return 0;
}

// Prompt of T tokens from an empty cache: embedding, every layer, final norm + lm_head + argmax of
// the last token (ids[0] then holds the first generated token).
int Session::prefill(const int* host_ids, int T) {
    CK(reserve(T));
    CK(hipMemcpyAsync(ids, host_ids, (size_t)T * 4, hipMemcpyHostToDevice, stream));
    CK(llm_embed(embed, ids, hidden, T, c.hidden, c.vocab_size, stream));
    CK(run_layers(T, 0));
    return last_token_logits(T, 0);
}

// Final norm of the last of T rows, lm_head and argmax: the token goes to ids[0] and
// tokens[step], and its embedding row to hidden row 0, the next decode step's input (the lm_head
// has read row T - 1 by then: same stream).
int Session::last_token_logits(int T, int step, int* state) {
    return llm_logits_argmax(c.layernorm != 0, hidden + (size_t)(T - 1) * c.hidden, fnorm, fnorm_b, c.norm_eps,
                             lm_head, logits, c.vocab_size, c.hidden, partial, scratch16, ids, tokens, step, stream,
                             state, embed, hidden);
}

// One decode step at cache position pos, token `step`: every layer over hidden row 0 (the
// previous argmax left the token's embedding there), final norm + lm_head + argmax. With dev, the
// kernels read the position and the token index from the device step state (and the argmax
// advances it), so the launches are the same for every step.
int Session::decode_step(int pos, int step, bool dev) {
    CK(run_layers(1, pos, dev ? dstate : nullptr));
    return last_token_logits(1, step, dev ? dstate : nullptr);
}

// The decode step as one graph launch (the ~5 launches per layer then cost ~1.9 us each instead
// of ~2.7 us as separate launches). The graph is captured on first use and again only when the
// attention plan changes with the cache length; dstate must hold {pos, step} for this step.
int Session::replay_step(int pos) {
    const cdna3_decode_cfg dc{c.head_dim, pos + 1, c.n_heads, c.n_kv_heads, 1, max_seq};
    const long long key = attn_decode_plan_key(dc);
    if (key < 0) return CDNA4_ERR_INVALID_VALUE;
    if (!gexec || key != gkey) {
        drop_graph();
        CK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
        const int e = decode_step(pos, 0, true);
        hipGraph_t g = nullptr;
        const hipError_t ee = hipStreamEndCapture(stream, &g);   // ends the capture on every path
        if (e != 0 || ee != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return e != 0 ? e : (int)ee;
        }
        graph = g;
        CK(hipGraphInstantiate(&gexec, graph, nullptr, nullptr, 0));
        gkey = key;
    }
    return (int)hipGraphLaunch(gexec, stream);
}

void Session::release() {
    if (stream) (void)hipStreamSynchronize(stream);
    drop_graph();
    for (void* ptr : scratch) (void)hipFree(ptr);
    for (void* ptr : allocs) (void)hipFree(ptr);
    scratch.clear();
    allocs.clear();
    if (blas) rocblas_destroy_handle(blas);
    if (stream) (void)hipStreamDestroy(stream);
    blas = nullptr;
    stream = nullptr;
}

}  // namespace cdna4

using namespace cdna4;

struct cdna3_session {
    Session impl;
};

extern "C" int cdna3_session_create(const char* model_dir, int max_seq, cdna3_session** out) {
    if (!model_dir || !out || max_seq < 1) return CDNA4_ERR_INVALID_VALUE;
    *out = nullptr;
    cdna3_session* s = nullptr;
    int e = 0;
    try {   // host allocations of the loader (file buffers, names) must not unwind through the C ABI
        s = new cdna3_session();
        s->impl.max_seq = max_seq;
        const char* g = getenv("CDNA4_SESSION_GRAPH");   // "0": separate launches per decode step
        s->impl.use_graph = !(g && g[0] == '0' && g[1] == 0);
        const char* rb = getenv("CDNA4_SESSION_ROCBLAS");
        s->impl.rocblas_only = rb && rb[0] == '1' && rb[1] == 0;
        const char* qf = getenv("CDNA4_SESSION_QKV_FUSED");
        s->impl.qkv_fused = !(qf && qf[0] == '0' && qf[1] == 0);
        const char* ap = getenv("CDNA4_SESSION_ATTN_PARTS");
        if (ap && ap[0] >= '0' && ap[0] <= '4' && ap[1] == 0) s->impl.attn_parts = ap[0] - '0';
        e = s->impl.read_config(model_dir);
        if (e == 0) e = check_device();
        if (e == 0) e = (int)hipStreamCreateWithFlags(&s->impl.stream, hipStreamNonBlocking);
        if (e == 0) e = s->impl.load(model_dir);
    } catch (const std::exception&) {
        e = (int)hipErrorOutOfMemory;
    }
    if (e != 0) {
        if (s) {
            s->impl.release();
            delete s;
        }
        return e;
    }
    *out = s;
    return 0;
}

extern "C" void cdna3_session_destroy(cdna3_session* s) {
    if (!s) return;
    s->impl.release();
    delete s;
}

extern "C" int cdna3_session_config(const cdna3_session* s, cdna3_model_cfg* out) {
    if (!s || !out) return CDNA4_ERR_INVALID_VALUE;
    *out = s->impl.c;
    return 0;
}

extern "C" int cdna3_session_generate(cdna3_session* s, const int* ids, int n_ids, int max_new_tokens,
                                      int eos_token_id, int* out_tokens, int* n_out, float* step_logits,
                                      float* ttft_ms, float* decode_ms) {
    if (!s || !ids || n_ids < 1 || max_new_tokens < 1 || !out_tokens || !n_out) return CDNA4_ERR_INVALID_VALUE;
    Session& S = s->impl;
    if (int e = S.check_ids(ids, n_ids)) return e;
    if (int e = check_device()) return e;
    *n_out = 0;
    // Decode step `step` writes cache row n_ids + step - 1; the reference stops once the cache
    // is full (session.hpp:283-284).
    if (max_new_tokens > S.max_seq - n_ids + 1) max_new_tokens = S.max_seq - n_ids + 1;
    CK(S.reserve(n_ids));   // before e0: a first call's allocations are not part of the timings
    hipEvent_t e0, e1, e2;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventCreate(&e2));
    int rc = 0;
    const size_t V = S.c.vocab_size;
    auto body = [&]() -> int {
        CK(hipEventRecord(e0, S.stream));
        CK(S.prefill(ids, n_ids));
        if (step_logits) CK(hipMemcpyAsync(step_logits, S.logits, V * 4, hipMemcpyDeviceToHost, S.stream));
        CK(hipEventRecord(e1, S.stream));
        int produced = 1;
        if (S.use_graph && max_new_tokens > 1) CK(llm_step_state(S.dstate, n_ids, 1, S.stream));
        for (int step = 1; step < max_new_tokens; ++step) {
            if (eos_token_id >= 0) {
                int last = -1;
                CK(hipMemcpyAsync(&last, S.ids, 4, hipMemcpyDeviceToHost, S.stream));
                CK(hipStreamSynchronize(S.stream));
                if (last == eos_token_id) break;
            }
            const int pos = n_ids + step - 1;
            if (S.use_graph) CK(S.replay_step(pos));
            else CK(S.decode_step(pos, step, false));
            if (step_logits)
                CK(hipMemcpyAsync(step_logits + (size_t)step * V, S.logits, V * 4, hipMemcpyDeviceToHost, S.stream));
            ++produced;
        }
        CK(hipEventRecord(e2, S.stream));
        CK(hipMemcpyAsync(out_tokens, S.tokens, (size_t)produced * 4, hipMemcpyDeviceToHost, S.stream));
        CK(hipStreamSynchronize(S.stream));
        *n_out = produced;
        float t = 0.f;
        CK(hipEventElapsedTime(&t, e0, e1));
        if (ttft_ms) *ttft_ms = t;
        CK(hipEventElapsedTime(&t, e1, e2));
        if (decode_ms) *decode_ms = t;
        return 0;
    };
    rc = body();
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipEventDestroy(e2);
    return rc;
}

extern "C" int cdna3_session_prefill_logits(cdna3_session* s, const int* ids, int n_ids, float* logits) {
    if (!s || !ids || !logits) return CDNA4_ERR_INVALID_VALUE;
    Session& S = s->impl;
    if (int e = S.check_ids(ids, n_ids)) return e;
    if (int e = check_device()) return e;
    CK(S.prefill(ids, n_ids));
    CK(hipMemcpyAsync(logits, S.logits, (size_t)S.c.vocab_size * 4, hipMemcpyDeviceToHost, S.stream));
    return (int)hipStreamSynchronize(S.stream);
}

// ---- ModelLoader: the model's tensors as the reference's loader leaves them ------------------------
// cdna3-prims/include/cdna3/runtime/model_loader.hpp:130-193: meta.json plus one raw fp16 .bin per
// tensor, each uploaded to its own device buffer under its own name (no concatenation; the session
// above builds its own fused layout instead). Optional q/k/v biases (qkv_bias) are NULL when absent.
struct cdna3_model {
    cdna3_model_cfg c{};
    std::vector<void*> allocs;
    std::vector<cdna3_layer_weights> layers;
    cdna3_model_weights view{};

    void release() {
        for (void* p : allocs) (void)hipFree(p);
        allocs.clear();
    }
    int upload(const std::string& path, size_t count, void** dst) {
        std::vector<uint16_t> h;
        if (!read_f16(path, count, h)) return CDNA4_ERR_INVALID_VALUE;
        CK(hipMalloc(dst, count * 2 ? count * 2 : 16));
        allocs.push_back(*dst);
        CK(hipMemcpy(*dst, h.data(), count * 2, hipMemcpyHostToDevice));
        return 0;
    }
    int load(const std::string& dir) {
        std::map<std::string, std::string> meta;
        if (!parse_meta(dir + "/meta.json", meta)) return CDNA4_ERR_INVALID_VALUE;
        auto geti = [&](const char* k, int def) { return meta.count(k) ? atoi(meta[k].c_str()) : def; };
        c.n_layers = geti("n_layers", 0);
        c.hidden = geti("hidden", 0);
        c.n_heads = geti("n_heads", 0);
        c.n_kv_heads = geti("n_kv_heads", c.n_heads);
        c.head_dim = geti("head_dim", c.n_heads ? c.hidden / c.n_heads : 0);
        c.ffn_dim = geti("ffn_dim", 0);
        c.vocab_size = geti("vocab_size", 0);
        c.rope_theta = meta.count("rope_theta") ? (float)atof(meta["rope_theta"].c_str()) : 10000.f;
        c.qkv_bias = meta.count("qkv_bias") && (meta["qkv_bias"] == "1" || meta["qkv_bias"] == "true");
        c.layernorm = meta.count("norm") && meta["norm"] == "layernorm";
        c.norm_eps = meta.count("norm_eps") ? (float)atof(meta["norm_eps"].c_str()) : (c.layernorm ? 1e-5f : 1e-6f);
        if (c.n_layers < 1 || c.hidden < 1 || c.n_heads < 1 || c.n_kv_heads < 1 || c.head_dim < 1 || c.ffn_dim < 1 ||
            c.vocab_size < 1)
            return CDNA4_ERR_INVALID_VALUE;
        const size_t H = c.hidden, F = c.ffn_dim, V = c.vocab_size;
        const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
        auto p = [&](const std::string& name) { return dir + "/" + name + ".bin"; };
        CK(upload(p("embed_tokens"), V * H, &view.embed_tokens));
        CK(upload(p("lm_head"), V * H, &view.lm_head));
        CK(upload(p("final_norm"), H, &view.final_norm));
        layers.assign(c.n_layers, cdna3_layer_weights{});
        for (int i = 0; i < c.n_layers; ++i) {
            const std::string lp = "layer_" + std::to_string(i) + "_";
            cdna3_layer_weights& l = layers[i];
            CK(upload(p(lp + "q_proj"), qd * H, &l.Wq));
            CK(upload(p(lp + "k_proj"), kvd * H, &l.Wk));
            CK(upload(p(lp + "v_proj"), kvd * H, &l.Wv));
            CK(upload(p(lp + "o_proj"), H * qd, &l.Wo));
            if (c.qkv_bias) {
                CK(upload(p(lp + "q_bias"), qd, &l.bq));
                CK(upload(p(lp + "k_bias"), kvd, &l.bk));
                CK(upload(p(lp + "v_bias"), kvd, &l.bv));
            }
            CK(upload(p(lp + "gate_proj"), F * H, &l.Wgate));
            CK(upload(p(lp + "up_proj"), F * H, &l.Wup));
            CK(upload(p(lp + "down_proj"), H * F, &l.Wdown));
            CK(upload(p(lp + "norm_attn"), H, &l.norm_attn));
            CK(upload(p(lp + "norm_mlp"), H, &l.norm_mlp));
        }
        view.n_layers = c.n_layers;
        view.layers = layers.data();
        return 0;
    }
};

extern "C" int cdna3_model_load(const char* model_dir, cdna3_model** out) {
    if (!model_dir || !out) return CDNA4_ERR_INVALID_VALUE;
    *out = nullptr;
    cdna3_model* m = nullptr;
    int e = 0;
    try {
        m = new cdna3_model();
        e = m->load(model_dir);
    } catch (const std::exception&) {
        e = (int)hipErrorOutOfMemory;
    }
    if (e != 0) {
        if (m) {
            m->release();
            delete m;
        }
        return e;
    }
    *out = m;
    return 0;
}

extern "C" void cdna3_model_free(cdna3_model* m) {
    if (!m) return;
    m->release();
    delete m;
}

extern "C" int cdna3_model_config(const cdna3_model* m, cdna3_model_cfg* out) {
    if (!m || !out) return CDNA4_ERR_INVALID_VALUE;
    *out = m->c;
    return 0;
}

extern "C" int cdna3_model_weights_get(const cdna3_model* m, cdna3_model_weights* out) {
    if (!m || !out) return CDNA4_ERR_INVALID_VALUE;
    *out = m->view;
    return 0;
}
