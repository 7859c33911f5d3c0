#pragma once
// dme:: 2-D tile prefetch and ping/pong buffers for gfx950.
//
// Names and arguments of the reference (research/dme-abstraction/include/dme/
// tensor_prefetch.hpp:64-196): prefetch_tile2d_fp16, prefetch_tile2d_strided_fp16,
// AsyncTile2D. The copies move 16 bytes per lane (global_load_lds_dwordx4) instead of 4, so a
// [kRows x kCols] fp16 tile needs kRows*kCols/8 lane copies. Participating threads must be
// whole waves (nthreads % 64 == 0, tid = wave * 64 + lane) and the tile row must be a whole
// number of 16-byte chunks (kCols % 8 == 0).
#include "dme_copy.hpp"
#include <hip/hip_fp16.h>

namespace dme {

template <int kRows, int kCols>
__device__ __forceinline__ void prefetch_tile2d_fp16(const __half* __restrict__ base_hbm, __half* __restrict__ dst_lds,
                                                     int tid, int nthreads) {
    static_assert(kCols % 8 == 0, "prefetch_tile2d_fp16: kCols must be a multiple of 8");
    constexpr int kChunks = kRows * kCols / 8;
    const int lane = tid & 63;
    for (int i = tid; i - lane < kChunks; i += nthreads) {   // wave-uniform trip count
        if (i < kChunks)                                          // lanes past the tile stay idle
            __builtin_amdgcn_global_load_lds((const void*)(base_hbm + (size_t)i * 8),
                                             (DME_LDS_AS void*)(dst_lds + (size_t)(i - lane) * 8), 16, 0, 1);
    }
}

template <int kRows, int kCols>
__device__ __forceinline__ void prefetch_tile2d_strided_fp16(const __half* __restrict__ base_hbm,
                                                             __half* __restrict__ dst_lds, int stride_row, int tid,
                                                             int nthreads) {
    static_assert(kCols % 8 == 0, "prefetch_tile2d_strided_fp16: kCols must be a multiple of 8");
    constexpr int kChunks = kRows * kCols / 8, kPerRow = kCols / 8;
    const int lane = tid & 63;
    for (int i = tid; i - lane < kChunks; i += nthreads) {
        if (i < kChunks) {
            const __half* src = base_hbm + (size_t)(i / kPerRow) * stride_row + (i % kPerRow) * 8;
            __builtin_amdgcn_global_load_lds((const void*)src, (DME_LDS_AS void*)(dst_lds + (size_t)(i - lane) * 8), 16,
                                             0, 1);
        }
    }
}

template <int kRows, int kCols>
struct AsyncTile2D {
    int cur_ = 0;
    __device__ __forceinline__ int cur() const { return cur_; }
    __device__ __forceinline__ int next() const { return cur_ ^ 1; }
    __device__ __forceinline__ void advance() { cur_ ^= 1; }

    __device__ __forceinline__ void prologue(const __half* __restrict__ base_hbm, __half dst_lds[][kRows * kCols],
                                             int tid, int nthreads) {
        prefetch_tile2d_fp16<kRows, kCols>(base_hbm, dst_lds[0], tid, nthreads);
        wait();
        __syncthreads();
        cur_ = 0;
    }
    __device__ __forceinline__ void prefetch_next(const __half* __restrict__ base_hbm, __half dst_lds[][kRows * kCols],
                                                  int next_tile_idx, int n_tiles, int tid, int nthreads) {
        if (next_tile_idx < n_tiles)
            prefetch_tile2d_fp16<kRows, kCols>(base_hbm + (size_t)next_tile_idx * kRows * kCols, dst_lds[next()], tid,
                                               nthreads);
    }
    __device__ __forceinline__ void wait_next(int /*next_tile_idx*/, int /*n_tiles*/) {
        wait();
        __syncthreads();
    }
};

}  // namespace dme
