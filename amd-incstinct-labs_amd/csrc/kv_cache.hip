// KV-cache append, layout repacks and the fused RoPE + append of the runtime layer loop (gfx950).
//
// Reference behaviour restated (cdna3-prims/include/cdna3/runtime/forward.hpp): scatter_kv_kernel
// (:209-220) writes token-major K/V [T][heads][D] into a head-major cache slot [heads][max_seq][D]
// at token offset pos0; repack_kernel (:190-205) converts [seq][heads][D] <-> [heads][seq][D];
// rope_kernel (:135-148) rotates halves (d, d + D/2) with cos/sin [seq][D]. The reference's layer
// loop (session.hpp:170-210) runs RoPE on Q and K, two scatters and up to four repacks per layer.
//
// MI355X design: these are pure HBM streams, so every kernel moves 16-byte vectors (8 fp16) per
// lane when D is a multiple of 8, and the fused entry point reads the token-major Q/K/V once and
// writes Q head-major plus the rotated K and the V rows into the cache in the same pass (one
// launch instead of seven). RoPE pairs (d, d + D/2) are handled by one lane each (the reference
// updates a pair from two threads in place, a read/write race).
#include "common.hpp"

namespace cdna4 {
namespace {

// cache[h][pos0 + s][:] = src[s][h][:], 16 bytes per lane (D % 8 == 0).
__global__ __launch_bounds__(256) void scatter_vec(const u32x4* __restrict__ src, u32x4* __restrict__ cache, int T,
                                                   int heads, int D, int pos0, int max_seq) {
    const int V = D / 8;
    const size_t total = (size_t)T * heads * V;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int v = (int)(i % V);
    const size_t sh = i / V;
    const int h = (int)(sh % heads);
    const int s = (int)(sh / heads);
    cache[((size_t)h * max_seq + pos0 + s) * V + v] = src[i];
}

__global__ __launch_bounds__(256) void scatter_elem(const uint16_t* __restrict__ src, uint16_t* __restrict__ cache,
                                                    int T, int heads, int D, int pos0, int max_seq) {
    const size_t total = (size_t)T * heads * D;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i % D);
    const size_t sh = i / D;
    const int h = (int)(sh % heads);
    const int s = (int)(sh / heads);
    cache[((size_t)h * max_seq + pos0 + s) * D + d] = src[i];
}

// dir 0: token-major [seq][heads][D] -> head-major [heads][seq][D]; dir 1: the reverse.
// Indexed by the token-major element, 16 bytes per lane when D % 8 == 0 (U = 8) else 2 (U = 1).
template <int U>
__global__ __launch_bounds__(256) void repack(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int seq,
                                              int heads, int D, int dir) {
    const int V = D / U;
    const size_t total = (size_t)seq * heads * V;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int v = (int)(i % V);
    const size_t sh = i / V;
    const int h = (int)(sh % heads);
    const int s = (int)(sh / heads);
    const size_t tok = i * U;
    const size_t hm = (((size_t)h * seq + s) * V + v) * U;
    const size_t from = dir == 0 ? tok : hm, to = dir == 0 ? hm : tok;
    if constexpr (U == 8) *(u32x4*)(dst + to) = *(const u32x4*)(src + from);
    else dst[to] = src[from];
}

// Fused RoPE + append. One lane per (token s, row slot r, pair j): slots [0, nQH) are query
// heads (rotated, written head-major to q_out [nQH][T][D]), [nQH, nQH + nKVH) key heads
// (rotated, into K_cache[h][pos0 + s]), the rest value heads (copied into V_cache[h][pos0 + s]).
__global__ __launch_bounds__(256) void rope_append(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                   const uint16_t* __restrict__ v, uint16_t* __restrict__ q_out,
                                                   uint16_t* __restrict__ Kc, uint16_t* __restrict__ Vc,
                                                   const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                   int T, int nQH, int nKVH, int D, int pos0, int max_seq,
                                                   long long ldq, long long ldk, long long ldv) {
    const int half = D >> 1;
    const int slots = nQH + 2 * nKVH;
    const size_t total = (size_t)T * slots * half;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int j = (int)(i % half);
    const size_t sr = i / half;
    const int r = (int)(sr % slots);
    const int s = (int)(sr / slots);
    const uint16_t* src;
    uint16_t* dst;
    bool rotate = true;
    if (r < nQH) {
        src = q + s * ldq + (size_t)r * D;
        dst = q_out + ((size_t)r * T + s) * D;
    } else if (r < nQH + nKVH) {
        const int h = r - nQH;
        src = k + s * ldk + (size_t)h * D;
        dst = Kc + ((size_t)h * max_seq + pos0 + s) * D;
    } else {
        const int h = r - nQH - nKVH;
        src = v + s * ldv + (size_t)h * D;
        dst = Vc + ((size_t)h * max_seq + pos0 + s) * D;
        rotate = false;
    }
    const uint32_t a = src[j], b = src[j + half];
    if (rotate) {
        const float* c = cosv + (size_t)s * D;
        const float* sn = sinv + (size_t)s * D;
        uint32_t lo, hi;
        rope_pair(a, b, c[j], sn[j], c[j + half], sn[j + half], lo, hi);
        dst[j] = (uint16_t)lo;
        dst[j + half] = (uint16_t)hi;
    } else {
        dst[j] = (uint16_t)a;
        dst[j + half] = (uint16_t)b;
    }
}

}  // namespace

// rope_append with explicit token strides (elements) of q, k and v, so the three can be column
// blocks of one [T][QD + 2 KVD] projection output. Arguments are validated by the caller.
int kv_rope_append(const void* q, const void* k, const void* v, long long ldq, long long ldk, long long ldv,
                   void* q_out, void* K_cache, void* V_cache, const float* cos_tab, const float* sin_tab, int T,
                   int nQH, int nKVH, int D, int pos0, int max_seq, hipStream_t stream) {
    const size_t total = (size_t)T * (nQH + 2 * nKVH) * (D / 2);
    rope_append<<<ceil_div(total, 256), 256, 0, stream>>>(
        (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)q_out, (uint16_t*)K_cache,
        (uint16_t*)V_cache, cos_tab, sin_tab, T, nQH, nKVH, D, pos0, max_seq, ldq, ldk, ldv);
    return launch_status();
}
}  // namespace cdna4

using namespace cdna4;

extern "C" int cdna3_scatter_kv_f16(const void* src, void* cache, int T, int heads, int D, int pos0, int max_seq,
                                    cdna4_stream_t stream) {
    if (T < 0 || heads < 1 || D < 1 || pos0 < 0 || (long long)pos0 + T > max_seq) return CDNA4_ERR_INVALID_VALUE;
    if (T == 0) return 0;
    if (!src || !cache) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    if (D % 8 == 0 && (((uintptr_t)src | (uintptr_t)cache) & 15u) == 0) {
        const size_t total = (size_t)T * heads * (D / 8);
        scatter_vec<<<ceil_div(total, 256), 256, 0, s>>>((const u32x4*)src, (u32x4*)cache, T, heads, D, pos0, max_seq);
    } else {
        const size_t total = (size_t)T * heads * D;
        scatter_elem<<<ceil_div(total, 256), 256, 0, s>>>((const uint16_t*)src, (uint16_t*)cache, T, heads, D, pos0,
                                                          max_seq);
    }
    return launch_status();
}

extern "C" int cdna3_repack_f16(const void* src, void* dst, int seq, int heads, int D, int dir,
                                cdna4_stream_t stream) {
    if (seq < 0 || heads < 1 || D < 1 || (dir != 0 && dir != 1)) return CDNA4_ERR_INVALID_VALUE;
    if (seq == 0) return 0;
    if (!src || !dst) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    hipStream_t s = (hipStream_t)stream;
    if (D % 8 == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0) {
        const size_t total = (size_t)seq * heads * (D / 8);
        repack<8><<<ceil_div(total, 256), 256, 0, s>>>((const uint16_t*)src, (uint16_t*)dst, seq, heads, D, dir);
    } else {
        const size_t total = (size_t)seq * heads * D;
        repack<1><<<ceil_div(total, 256), 256, 0, s>>>((const uint16_t*)src, (uint16_t*)dst, seq, heads, D, dir);
    }
    return launch_status();
}

extern "C" int cdna3_rope_append_kv_f16(const void* q, const void* k, const void* v, void* q_out, void* K_cache,
                                        void* V_cache, const float* cos_tab, const float* sin_tab, int T, int nQH,
                                        int nKVH, int D, int pos0, int max_seq, cdna4_stream_t stream) {
    if (T < 0 || nQH < 1 || nKVH < 1 || D < 2 || (D & 1) || pos0 < 0 || (long long)pos0 + T > max_seq)
        return CDNA4_ERR_INVALID_VALUE;
    if (T == 0) return 0;
    if (!q || !k || !v || !q_out || !K_cache || !V_cache || !cos_tab || !sin_tab) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    return kv_rope_append(q, k, v, (long long)nQH * D, (long long)nKVH * D, (long long)nKVH * D, q_out, K_cache,
                          V_cache, cos_tab, sin_tab, T, nQH, nKVH, D, pos0, max_seq, (hipStream_t)stream);
}
