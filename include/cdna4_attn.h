/*
 * cdna4_attn.h — C ABI of libcdna4_attn.so, the MI355X (gfx950) attention hot path.
 *
 * Plain C: device pointers, sizes, plain structs and a stream handle. No C++ or torch
 * types cross this boundary. Every entry point:
 *   - enqueues its kernels on `stream` (NULL = the default stream) and returns without
 *     synchronising;
 *   - returns 0 (hipSuccess) or a hipError_t value: CDNA4_ERR_INVALID_VALUE (1) for a
 *     shape, dtype or op it does not support, CDNA4_ERR_INVALID_DEVICE_FUNCTION (98)
 *     when the current device is not gfx950, otherwise the launch error;
 *   - never allocates device memory and keeps no device buffers between calls (the session
 *     API below owns the memory of its session);
 * Entry points are re-entrant from any host thread, ordering coming from the stream, with one
 * exception: cdna3_attn_decode_noalloc, whose calls on one GPU share a static device array, so
 * calls of it that overlap on one GPU race (see its declaration). A caller's workspace or
 * session must likewise not be used by calls that overlap.
 *
 * Tensor layouts are row-major and contiguous unless a stride is given.
 */
#ifndef CDNA4_ATTN_H
#define CDNA4_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is `struct ihipStream_t*`; this typedef is layout-identical. */
typedef struct ihipStream_t* cdna4_stream_t;

#define CDNA4_ABI_VERSION 2

enum {
    CDNA4_OK = 0,
    CDNA4_ERR_INVALID_VALUE = 1,
    CDNA4_ERR_SCRATCH_TOO_SMALL = 0x4344,  /* outside the hipError_t range: the call needs more
                                              than the static scratch of
                                              cdna3_attn_decode_noalloc holds */
    CDNA4_ERR_INVALID_DEVICE_FUNCTION = 98
};

/* Element types. */
enum {
    CDNA4_F32 = 0,
    CDNA4_F16 = 1,
    CDNA4_BF16 = 2,
    CDNA4_F64 = 3,
    CDNA4_I32 = 4,
    CDNA4_I64 = 5
};

/* Reduction / scan operators. */
enum {
    CDNA4_OP_SUM = 0,
    CDNA4_OP_MAX = 1,
    CDNA4_OP_MIN = 2
};

/* Field for field the reference's cdna3::attn::PrefillCfg
 * (cdna3-prims/include/cdna3/attention.hpp:63-71). */
typedef struct {
    int D;         /* head dimension: 64 or 128 */
    int seqQ;      /* query rows per (batch, head) */
    int seqK;      /* key/value rows per (batch, kv head) */
    int nQHeads;
    int nKVHeads;  /* nQHeads % nKVHeads == 0 (GQA) */
    int batch;
    int causal;    /* 1: key k visible to query q iff k <= q (requires seqQ == seqK) */
} cdna3_prefill_cfg;

/* The reference's DecodeCfg {D, N, nQHeads, nKVHeads} (attention.hpp:73-78) and
 * DecodeDmeCfg {.., stride_kv} (detail/fa_decode_dme_kernel.hpp:45-48), plus batch. */
typedef struct {
    int D;          /* 64 or 128 */
    int N;          /* cached keys per sequence */
    int nQHeads;
    int nKVHeads;
    int batch;      /* >= 1 */
    int stride_kv;  /* rows between kv heads in K/V; 0 or N = packed; >= N otherwise */
} cdna3_decode_cfg;

/* ---- library ---------------------------------------------------------------- */

/* ABI version of the loaded library (CDNA4_ABI_VERSION it was built with). */
int cdna3_abi_version(void);

/* Static text for a return code of this library. */
const char* cdna3_error_string(int code);

/* ---- attention: prefill ------------------------------------------------------
 * Replaces cdna3::attn::prefill (cdna3-prims/include/cdna3/attention.hpp:86-109).
 * Q, O: [batch][nQHeads][seqQ][D]; K, V: [batch][nKVHeads][seqK][D]; dtype is
 * CDNA4_F16, CDNA4_BF16 or CDNA4_F32 for all four. Scale 1/sqrt(D), softmax and
 * accumulation in fp32. Query head h reads kv head h / (nQHeads / nKVHeads).
 * Unlike the reference, any seqQ, seqK >= 1 is accepted (ragged tails are masked);
 * shapes the reference would silently truncate therefore compute the full result.
 * Invalid: D not in {64,128}, non-positive sizes, nQHeads % nKVHeads != 0,
 * causal with seqQ != seqK, an unknown dtype, Q/K/V not 16-byte aligned, O not 8-byte
 * (16-bit) or 4-byte (fp32) aligned.
 */
int cdna3_attn_prefill(const void* Q, const void* K, const void* V, void* O,
                       const cdna3_prefill_cfg* cfg, int dtype, cdna4_stream_t stream);

/*
 * cdna3_attn_prefill_strided: the same computation with explicit element strides, so a caller
 * can attend over tensors that are not packed [batch][heads][seq][D]: e.g. K/V read in place
 * from a KV cache [nKVH][max_seq][D] (kv_head = max_seq * D) and O written token-major
 * [seq][nQH][D] (o_head = D, o_row = nQH * D) for the projection that follows. No counterpart
 * in the reference, whose layer loop repacked Q, K, V and O around the call
 * (cdna3-prims/include/cdna3/runtime/session.hpp:190-207). dtype f16 or bf16; every Q/K/V
 * stride a multiple of 8 elements and every O stride a multiple of 4; rows no shorter than D.
 */
typedef struct cdna3_prefill_strides {
    long long q_batch, q_head, q_row;     /* Q element strides */
    long long kv_batch, kv_head, kv_row;  /* K and V element strides */
    long long o_batch, o_head, o_row;     /* O element strides */
} cdna3_prefill_strides;

int cdna3_attn_prefill_strided(const void* Q, const void* K, const void* V, void* O,
                               const cdna3_prefill_cfg* cfg,
                               const cdna3_prefill_strides* strides, int dtype,
                               cdna4_stream_t stream);

/* ---- attention: decode (one query per sequence, split-K) --------------------
 * Replaces cdna3::attn::decode (attention.hpp:117-137) and cdna3::attn::decode_dme
 * (attention.hpp:152-173); the reference has no batch dimension (batch == 1 here).
 * q, o: [batch][nQHeads][D]; K, V: [batch][nKVHeads][stride_kv][D] (first N rows of
 * each head are read). dtype CDNA4_F16 or CDNA4_BF16 (q, K, V, o alike).
 * With a workspace (ws_bytes >= cdna3_attn_decode_workspace_size(cfg); the contents need no
 * initialisation), long caches are split over a grid of single-wave workgroups that leave
 * (m, l, O) partials in it, merged by a second kernel, unless batch x nKVHeads x (groups of 16
 * query heads) is a multiple of the device's CU count: then the one-launch plan below fills
 * whole rounds of the CUs and is taken instead (the workspace is then not used). With
 * workspace == NULL the call takes
 * the one-launch plan, which needs no memory beyond q, K, V and o: one workgroup per (batch,
 * kv head, group of 16 query heads) streams the whole cache, like the reference's launchers,
 * which take no workspace. Both forms are capturable and re-entrant across streams (a
 * workspace must not be shared by calls that overlap). CDNA4_DECODE_SPLIT_K=1 in the environment
 * (read on every call, by the workspace-size and plan queries too) keeps calls with a workspace
 * on the split-K plan at whole rounds of CUs as well, to time the two plans against each other.
 */
size_t cdna3_attn_decode_workspace_size(const cdna3_decode_cfg* cfg);
int cdna3_attn_decode(const void* q, const void* K, const void* V, void* o,
                      const cdna3_decode_cfg* cfg, int dtype,
                      void* workspace, size_t ws_bytes, cdna4_stream_t stream);

/*
 * cdna3_attn_decode_noalloc: no counterpart in the reference. For callers that cannot allocate
 * (code under HIP graph capture that must not call hipMalloc, tight serving loops, harnesses that
 * forbid allocation): the computation of cdna3_attn_decode with a workspace, with its split-K
 * partials (when its plan has any) in a static device array of the library (cdna3_attn_decode_noalloc_max_bytes(), 16 MiB
 * per GPU, held until the process ends) instead of a caller's workspace. The caller passes only
 * q, K, V and o; the call never allocates. Returns CDNA4_ERR_SCRATCH_TOO_SMALL when the plan's
 * partials (cdna3_attn_decode_workspace_size(cfg)) exceed the array. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (concurrent streams, or host threads launching
 * on different streams) race and must be serialised by the caller.
 */
size_t cdna3_attn_decode_noalloc_max_bytes(void);
int cdna3_attn_decode_noalloc(const void* q, const void* K, const void* V, void* o,
                              const cdna3_decode_cfg* cfg, int dtype, cdna4_stream_t stream);

/* ---- kernel plans (introspection) ---------------------------------------------
 * No counterpart in the reference (its launchers had one kernel each). Report which kernel a
 * call with the same arguments would launch on the current device, without launching it, so
 * tests and profilers can assert the kernel they mean to cover. Returns 0 or
 * CDNA4_ERR_INVALID_VALUE for arguments the entry point would reject.
 */
enum {
    CDNA4_KERNEL_PREFILL_MFMA_8W = 1,  /* fa_mfma: 8 waves x 32 queries, persistent XCD-local grid */
    CDNA4_KERNEL_PREFILL_MFMA_4W = 2,  /* fa_mfma: 4 waves x 16 queries, one workgroup per block */
    CDNA4_KERNEL_PREFILL_SMALL = 3,    /* fa_small: 16 queries per workgroup, keys split over its waves */
    CDNA4_KERNEL_PREFILL_F32 = 4,      /* fa_f32: fp32 matrix-core kernel */
    CDNA4_KERNEL_DECODE_SPLIT = 5,     /* decode_mfma split-K grid + decode_merge */
    CDNA4_KERNEL_DECODE_WG = 6         /* decode_wg: one launch, no workspace */
};

typedef struct {
    int kernel;        /* CDNA4_KERNEL_* */
    int waves;         /* waves per workgroup */
    int rows;          /* prefill: query rows per work item; decode: keys per split (per wave for WG) */
    int partials;      /* decode: split-K partials per query head (1 for one launch); prefill: 1 */
    long long grid;    /* workgroups launched */
    size_t workspace;  /* bytes of workspace the plan needs (0: none) */
} cdna3_plan_info;

int cdna3_attn_prefill_plan(const cdna3_prefill_cfg* cfg, int dtype, cdna3_plan_info* out);
int cdna3_attn_decode_plan(const cdna3_decode_cfg* cfg, int dtype, int with_workspace,
                           cdna3_plan_info* out);

/* ---- device-wide reduce / scan on the wave64 DPP primitives ------------------
 * Device-wide counterparts of wave::dpp::reduce_* / scan_inclusive_* (research/
 * wave-primitives/include/wave_primitives/wave_reduce_dpp.hpp:106-113,
 * wave_scan_dpp.hpp:70-87), which exist only at wave level in the reference.
 * dtype: CDNA4_F32, F64, I32, I64 (result type = input type) or CDNA4_F16 / BF16
 * (fp32 accumulation, fp32 result). Integer sums wrap in two's complement.
 * reduce: `out` receives one element. scan: `out` receives n elements.
 * n == 0: reduce writes the operator's identity; scan writes nothing.
 * Workspace: >= the returned size. The scan's look-back flags carry a per-call epoch, so a
 * workspace needs no clearing between calls (one launch per call, plus a one-wave tail launch
 * for the last n % 4 elements of an aligned call). A zeroed workspace, or one last used by
 * another scan, is always safe; memory never written by a scan is accepted too, with the caveat
 * that a 64-bit word of it whose upper half happens to equal the call's 32-bit tag would be read
 * as published (so zero a fresh workspace once to rule that out).
 * Scan status: the scan's decoupled look-back waits a bounded time for a predecessor tile; if a
 * wait ever exceeds that bound the result is not valid and the call marks the workspace
 * (its first word takes the call's epoch, the second word holds the epoch of the latest call).
 * cdna3_scan_status synchronises `stream` and returns 1 in *status when the latest scan on this
 * workspace gave up a wait, else 0.
 * The bound is 2^22 sleeps per wait; CDNA4_SCAN_SPIN_LIMIT in the environment (read on every
 * call) lowers it, so that tests can force the timeout path.
 */
size_t cdna3_reduce_workspace_size(size_t n, int dtype);
int cdna3_reduce(int op, int dtype, const void* in, size_t n, void* out,
                 void* workspace, size_t ws_bytes, cdna4_stream_t stream);
size_t cdna3_scan_workspace_size(size_t n, int dtype);
int cdna3_scan_inclusive(int op, int dtype, const void* in, size_t n, void* out,
                         void* workspace, size_t ws_bytes, cdna4_stream_t stream);
int cdna3_scan_status(const void* workspace, int* status, cdna4_stream_t stream);

/* ---- row softmax ---------------------------------------------------------------
 * cdna3_softmax_rows_f32 replaces softmax_kernel<DPP> (research/wave-primitives/benchmarks/
 * bench_softmax.hip:59-105, launched there with one 64-lane block per row of 64 x ELEMS_PER_LANE
 * columns): Y[r][c] = exp(X[r][c] - max_c X[r]) / sum_c exp(X[r][c] - max_c X[r]) for M rows of
 * H fp32 values, any H >= 1 (the reference's kernel fixed H at compile time); X may equal Y.
 * Invalid: M < 0, H < 1, null pointers with M > 0.
 */
int cdna3_softmax_rows_f32(const float* X, float* Y, int M, int H, cdna4_stream_t stream);

/* ---- runtime norms and RoPE ---------------------------------------------------
 * cdna3_rmsnorm_f32 replaces rmsnorm_f32_kernel (cdna3-prims/include/cdna3/runtime/
 * forward.hpp:34-56): Y[m][i] = X[m][i] * rsqrt(mean_i(X[m][:]^2) + eps) * W[i],
 * X, Y fp32 [M][H], W fp16 [H]. Any H >= 1.
 * cdna3_layernorm_f32 replaces the two-pass DPP layernorm_kernel (research/
 * wave-primitives/benchmarks/bench_layernorm.hip:51-114) with runtime H:
 * Y = (X - mean) * rsqrt(var + eps) * gamma + beta, var = mean((X - mean)^2).
 * cdna3_rope_f16 replaces rope_kernel (forward.hpp:135-148): rotate-half RoPE in place
 * on T fp16 [seq][heads][D] with cos/sin fp32 [seq][D]; each (d, d+D/2) pair is read
 * and written by one thread (the reference updates the pair from two threads).
 * cdna3_rope_table_f32 fills cos/sin [T][D] for positions pos0.. on the device, as the
 * host loop Session::fill_rope does (cdna3-prims/include/cdna3/runtime/session.hpp:
 * 120-135): freq_d = theta^(-2d/D), entries d and d + D/2 share angle pos * freq_d.
 */
int cdna3_rmsnorm_f32(const float* X, const void* W_f16, float* Y, int M, int H,
                      float eps, cdna4_stream_t stream);
int cdna3_layernorm_f32(const float* X, const float* gamma, const float* beta, float* Y,
                        int M, int H, float eps, cdna4_stream_t stream);
int cdna3_rope_f16(void* T, const float* cos_tab, const float* sin_tab, int seq,
                   int heads, int D, cdna4_stream_t stream);
int cdna3_rope_table_f32(float* cos_tab, float* sin_tab, int pos0, int T, int D,
                         float theta, cdna4_stream_t stream);

/*
 * The runtime's prompt GEMM: Y[M][N] = X[M][K] W[N][K]^T (+ Y when accum = 1), X and W fp16
 * row-major, fp32 accumulation, Y fp32 (y_f32 = 1) or fp16 with leading dimension ldy. It
 * replaces, for the shapes it takes, the rocBLAS gemm_ex call of the reference's runtime
 * (cdna3-prims/include/cdna3/runtime/rocblas_gemm.hpp:8-20, forward.hpp:70-131; beta 0 or 1).
 * Returns CDNA4_ERR_INVALID_VALUE, launching nothing, when K is not a multiple of 64, N or ldy
 * not a multiple of 4, ldy < N, X or W not 16-byte aligned or Y not 16- (fp32) or 8-byte (fp16)
 * aligned (the session then calls rocBLAS).
 */
int cdna4_gemm_f16_nt(const void* X, const void* W, void* Y, int y_f32, int accum, int M, int N,
                      int K, int ldy, cdna4_stream_t stream);
/* The BM x BN tile (rows of X x rows of W per workgroup) cdna4_gemm_f16_nt takes for a shape on
 * the current device (no counterpart in the reference: tests use it to cover every tile). */
int cdna4_gemm_f16_nt_tile(int M, int N, int K, int* bm, int* bn);
/* The SwiGLU gate|up product and the SiLU product in one launch: W = [Wg; Wu] fp16 [2F][K]
 * (gate rows, then up rows), Y fp16 [M][F] (leading dimension ldy) = fp16(silu(g) * u) with
 * g = X Wg^T and u = X Wu^T accumulated in fp32. Replaces the reference runtime's gate and up
 * GEMMs followed by silu_mul_f32_kernel (cdna3-prims/include/cdna3/runtime/session.hpp:227-231,
 * forward.hpp:154-160). Same shape rules as cdna4_gemm_f16_nt (F a multiple of 4, Y 8-byte
 * aligned); cdna4_gemm_f16_nt_silu_tile reports its tile (BN counts gate and up rows). */
int cdna4_gemm_f16_nt_silu(const void* X, const void* W, void* Y, int M, int F, int K, int ldy,
                           cdna4_stream_t stream);
int cdna4_gemm_f16_nt_silu_tile(int M, int F, int K, int* bm, int* bn);

/*
 * KV cache and layout kernels of the runtime layer loop (all fp16, device pointers).
 * cdna3_scatter_kv_f16 replaces scatter_kv_kernel (cdna3-prims/include/cdna3/runtime/
 * forward.hpp:209-220, launched by Session::append_kv, session.hpp:240-250):
 * cache[h][pos0 + s][d] = src[s][h][d] for s < T, cache [heads][max_seq][D]; requires
 * pos0 + T <= max_seq (the reference wrote past the slot otherwise).
 * cdna3_repack_f16 replaces repack_kernel (forward.hpp:190-205): dir 0 turns token-major
 * [seq][heads][D] into head-major [heads][seq][D], dir 1 the reverse.
 * cdna3_rope_append_kv_f16 fuses what the reference's layer loop does with two rope_kernel
 * launches, append_kv and the Q repack (session.hpp:170-199): q, k, v are token-major
 * [T][nQH][D], [T][nKVH][D], [T][nKVH][D]; it writes rotate-half RoPE(q) head-major to
 * q_out [nQH][T][D], RoPE(k) to K_cache[h][pos0 + s] and v to V_cache[h][pos0 + s]
 * ([nKVH][max_seq][D] caches), with cos/sin [T][D] for positions pos0 .. pos0 + T - 1
 * (cdna3_rope_table_f32). Inputs are not modified.
 */
int cdna3_scatter_kv_f16(const void* src, void* cache, int T, int heads, int D, int pos0,
                         int max_seq, cdna4_stream_t stream);
int cdna3_repack_f16(const void* src, void* dst, int seq, int heads, int D, int dir,
                     cdna4_stream_t stream);
int cdna3_rope_append_kv_f16(const void* q, const void* k, const void* v, void* q_out,
                             void* K_cache, void* V_cache, const float* cos_tab,
                             const float* sin_tab, int T, int nQH, int nKVH, int D, int pos0,
                             int max_seq, cdna4_stream_t stream);

/* ---- small-LLM runtime session ------------------------------------------------
 * Replaces cdna3::runtime::Session (cdna3-prims/include/cdna3/runtime/session.hpp:47-331) with
 * its ModelLoader (model_loader.hpp:130-193) and KVCache (kv_cache.hpp:19-52): greedy batch-1
 * generation over a decoder read from the reference's export format, a directory holding
 * meta.json (flat keys n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size,
 * rope_theta, qkv_bias) and one raw little-endian fp16 .bin per tensor: embed_tokens,
 * lm_head [vocab][hidden], final_norm [hidden], layer_<i>_{q,k,v,o,gate,up,down}_proj
 * (row-major [out][in]), layer_<i>_{q,k,v}_bias when qkv_bias, layer_<i>_norm_{attn,mlp}.
 * Extensions (absent keys keep the reference's behaviour): "norm": "layernorm" selects two-pass
 * LayerNorm (eps 1e-5) instead of RMSNorm (eps 1e-6), with optional *_norm_*_bias /
 * final_norm_bias tensors as beta; "norm_eps" overrides eps.
 * Numerics follow the reference: fp32 residual stream, fp16 activations into each projection
 * with fp32 accumulation, fp16 Q/K/V and KV cache, fp32 SiLU product; logits are accumulated in
 * fp32 and stored as fp16 (returned widened to fp32), and the greedy argmax breaks ties as the
 * reference's argmax_kernel does (forward.hpp:244-262, a 256-thread strided scan and tree
 * reduction): among equal maxima, the index i with the smallest bit-reversed (i mod 256) as an
 * 8-bit number, then the smallest i / 256.
 * The session owns one HIP stream, a rocBLAS handle, the weights and the KV cache
 * [layers][n_kv_heads][max_seq][head_dim]. Calls on one session must not overlap.
 */
typedef struct cdna3_session cdna3_session;

typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size;
    float rope_theta;
    int qkv_bias;    /* 1: per-layer q/k/v biases */
    int layernorm;   /* 1: LayerNorm, 0: RMSNorm */
    float norm_eps;
} cdna3_model_cfg;

/* Session(model_dir, max_seq) (session.hpp:254-260): loads the model onto the current device.
 * Invalid: unreadable or short files, head_dim not 64/128, n_heads % n_kv_heads != 0, hidden or
 * ffn_dim not a multiple of 8, hidden > 4096. */
int cdna3_session_create(const char* model_dir, int max_seq, cdna3_session** out);
void cdna3_session_destroy(cdna3_session* session);
int cdna3_session_config(const cdna3_session* session, cdna3_model_cfg* out);

/* Session::generate (session.hpp:262-296): prefill ids[0..n_ids), then greedy decode. Writes
 * the generated tokens only (the reference returns the prompt followed by them) to out_tokens
 * (room for max_new_tokens) and their count to *n_out. Stops after an eos_token_id (>= 0) has
 * been produced, or when the cache is full (n_ids + steps == max_seq), as the reference does.
 * Optional outputs (NULL to skip): step_logits, host [max_new_tokens][vocab] logits (fp16 values as fp32) of each
 * step; ttft_ms, device time from the prompt upload to the first token; decode_ms, device time
 * of the remaining steps. Invalid: n_ids < 1 or > max_seq, ids out of [0, vocab). */
int cdna3_session_generate(cdna3_session* session, const int* ids, int n_ids, int max_new_tokens,
                           int eos_token_id, int* out_tokens, int* n_out, float* step_logits,
                           float* ttft_ms, float* decode_ms);

/* Session::prefill_logits (session.hpp:298-317): prefill only; host logits [vocab] of the last
 * prompt token (the fp16 values, widened to fp32, as the reference returns them). */
int cdna3_session_prefill_logits(cdna3_session* session, const int* ids, int n_ids,
                                 float* logits);

/* ---- model loader ----------------------------------------------------------------
 * Replaces cdna3::runtime::ModelLoader (cdna3-prims/include/cdna3/runtime/model_loader.hpp:
 * 130-193): reads the same directory format as cdna3_session_create and uploads every tensor to
 * its own fp16 device buffer on the current device, under the reference's names (q/k/v biases
 * NULL unless qkv_bias). The buffers stay valid until cdna3_model_free. Invalid: unreadable
 * meta.json, non-positive sizes, missing or short tensor files.
 */
typedef struct cdna3_model cdna3_model;

typedef struct {
    void *Wq, *Wk, *Wv, *Wo;     /* [n_heads*head_dim][hidden], [n_kv*hd][hidden] x2, [hidden][n_heads*hd] */
    void *bq, *bk, *bv;          /* NULL without qkv_bias */
    void *Wgate, *Wup, *Wdown;   /* [ffn][hidden] x2, [hidden][ffn] */
    void *norm_attn, *norm_mlp;  /* [hidden] */
} cdna3_layer_weights;

typedef struct {
    void* embed_tokens;                 /* [vocab][hidden] */
    void* lm_head;                      /* [vocab][hidden] */
    void* final_norm;                   /* [hidden] */
    int n_layers;
    const cdna3_layer_weights* layers;  /* n_layers entries, owned by the model */
} cdna3_model_weights;

int cdna3_model_load(const char* model_dir, cdna3_model** out);
void cdna3_model_free(cdna3_model* model);
int cdna3_model_config(const cdna3_model* model, cdna3_model_cfg* out);
int cdna3_model_weights_get(const cdna3_model* model, cdna3_model_weights* out);

#ifdef __cplusplus
}
#endif

#endif /* CDNA4_ATTN_H */
