#pragma once
// dme:: asynchronous HBM -> LDS copies for gfx950 (global_load_lds), wave64.
//
// API of the reference's "DME" wrapper (research/dme-abstraction/include/dme/dme_copy.hpp:
// 63-146): copy_element(_stream), copy_tile_1d(_stream), wait, wait_lds. On gfx950 the same
// instruction family also moves 16 bytes per lane (global_load_lds_dwordx4), which this build
// adds as copy16 / copy_tile_16B: one instruction moves 1 KiB per wave.
//
// Semantics checked on an MI355X: the LDS destination of lane L is (wave-uniform base) +
// L * size; each lane supplies its own global source address. Callers therefore pass the
// wave's base LDS address (identical on all 64 lanes) and per-lane sources. The copy is
// tracked by vmcnt: wait() (s_waitcnt 0) before reading the data, plus a barrier when other
// waves read it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dme {

#define DME_LDS_AS __attribute__((address_space(3)))

__device__ __forceinline__ unsigned lane_id() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// 4-byte per-lane copy into (wave base of dst_lds) + lane * 4 (reference API; dst_lds is this
// lane's slot, from which the wave base is derived).
template <typename T>
__device__ __forceinline__ void copy_element(const T* __restrict__ src_global, T* __restrict__ dst_lds) {
    static_assert(sizeof(T) == 4, "copy_element: T must be 4 bytes");
    __builtin_amdgcn_global_load_lds((const void*)src_global, (DME_LDS_AS void*)(dst_lds - lane_id()), 4, 0, 0);
}
// Streaming variant: non-temporal hint (aux bit 1), data not expected to be re-read from cache.
template <typename T>
__device__ __forceinline__ void copy_element_stream(const T* __restrict__ src_global, T* __restrict__ dst_lds) {
    static_assert(sizeof(T) == 4, "copy_element_stream: T must be 4 bytes");
    __builtin_amdgcn_global_load_lds((const void*)src_global, (DME_LDS_AS void*)(dst_lds - lane_id()), 4, 0, 1);
}

// 16-byte per-lane copy: lane L's 16 bytes land at dst_wave_base + 16 * L.
__device__ __forceinline__ void copy16(const void* src_global, void* dst_wave_base) {
    __builtin_amdgcn_global_load_lds(src_global, (DME_LDS_AS void*)dst_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void copy16_stream(const void* src_global, void* dst_wave_base) {
    __builtin_amdgcn_global_load_lds(src_global, (DME_LDS_AS void*)dst_wave_base, 16, 0, 1);
}

__device__ __forceinline__ void wait() { __builtin_amdgcn_s_waitcnt(0); }
// LDS-side counter only (reference wait_lds, dme_copy.hpp:97-99).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// One wave copies kElems 4-byte elements (kElems % 64 == 0), element i -> dst_lds[i].
template <typename T, int kElems>
__device__ __forceinline__ void copy_tile_1d(const T* __restrict__ src, T* __restrict__ dst_lds) {
    static_assert(sizeof(T) == 4, "copy_tile_1d: T must be 4 bytes");
    static_assert(kElems % 64 == 0, "copy_tile_1d: kElems must be a multiple of 64");
    const unsigned lane = lane_id();
#pragma unroll
    for (int i = 0; i < kElems / 64; ++i)
        __builtin_amdgcn_global_load_lds((const void*)(src + i * 64 + lane), (DME_LDS_AS void*)(dst_lds + i * 64), 4, 0, 0);
}
template <typename T, int kElems>
__device__ __forceinline__ void copy_tile_1d_stream(const T* __restrict__ src, T* __restrict__ dst_lds) {
    static_assert(sizeof(T) == 4, "copy_tile_1d_stream: T must be 4 bytes");
    static_assert(kElems % 64 == 0, "copy_tile_1d_stream: kElems must be a multiple of 64");
    const unsigned lane = lane_id();
#pragma unroll
    for (int i = 0; i < kElems / 64; ++i)
        __builtin_amdgcn_global_load_lds((const void*)(src + i * 64 + lane), (DME_LDS_AS void*)(dst_lds + i * 64), 4, 0, 1);
}

// One wave copies kBytes (kBytes % 1024 == 0) with 16-byte lanes: byte i -> dst_lds + i.
template <int kBytes>
__device__ __forceinline__ void copy_tile_16B(const void* __restrict__ src, void* __restrict__ dst_lds) {
    static_assert(kBytes % 1024 == 0, "copy_tile_16B: kBytes must be a multiple of 1024");
    const unsigned lane = lane_id();
    const char* s = (const char*)src;
    char* d = (char*)dst_lds;
#pragma unroll
    for (int i = 0; i < kBytes / 1024; ++i) copy16(s + i * 1024 + lane * 16, d + i * 1024);
}

}  // namespace dme
