#pragma once
// wave::dpp prefix scans for gfx950 (CDNA4), wave64, zero LDS instructions.
//
// Same names and semantics as the reference's wave::dpp scans
// (research/wave-primitives/include/wave_primitives/wave_scan_dpp.hpp:31-87):
//   scan_inclusive(v, op, identity), scan_inclusive_sum / _max / _min,
//   scan_exclusive_sum, scan_id_*, ScanSum / ScanMax / ScanMin, scan_lane_id, scan_dpp_step.
// The in-row part (row_shr 1/2/4/8) is the same Hillis-Steele step the reference
// uses; the cross-row carry is re-derived for gfx950 from row_newbcast:15 and the
// permlane16/32 swaps (detail/xlane.hpp) instead of three cascaded row_bcast15.
//
// New in this build: scan_exclusive (any op), and fp16 / bf16 inputs that
// accumulate in fp32 and return float.
#include "detail/xlane.hpp"
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <hip/hip_bfloat16.h>

namespace wave {
namespace dpp {

template <typename T> __device__ __forceinline__ T scan_id_sum() { return T(0); }
template <typename T> __device__ __forceinline__ T scan_id_max() { return std::numeric_limits<T>::lowest(); }
template <typename T> __device__ __forceinline__ T scan_id_min() { return std::numeric_limits<T>::max(); }

using ScanSum = xlane::Sum;
using ScanMax = xlane::Max;
using ScanMin = xlane::Min;

__device__ __forceinline__ unsigned scan_lane_id() { return xlane::lane(); }

// One in-row Hillis-Steele step: op(v, the value Shift lanes below within the 16-lane row), lanes
// with no such neighbour combining with `identity` (row_shr:Shift, Shift in 1, 2, 4, 8).
template <int Shift, typename T, typename Op>
__device__ __forceinline__ T scan_dpp_step(T v, Op op, T identity) {
    static_assert(Shift == 1 || Shift == 2 || Shift == 4 || Shift == 8, "row_shr 1/2/4/8");
    const T moved = xlane::dpp<0x110 + Shift>(identity, v);
    return op(v, moved);
}

// The identity argument is kept for signature compatibility; Op supplies its own.
template <typename T, typename Op>
__device__ __forceinline__ T scan_inclusive(T v, Op op, T /*identity*/) {
    return xlane::scan_inclusive(v, op);
}

template <typename T> __device__ __forceinline__ T scan_inclusive_sum(T v) { return xlane::scan_inclusive(v, ScanSum{}); }
template <typename T> __device__ __forceinline__ T scan_inclusive_max(T v) { return xlane::scan_inclusive(v, ScanMax{}); }
template <typename T> __device__ __forceinline__ T scan_inclusive_min(T v) { return xlane::scan_inclusive(v, ScanMin{}); }
template <typename T> __device__ __forceinline__ T scan_exclusive_sum(T v) { return xlane::scan_exclusive(v, ScanSum{}); }
template <typename T, typename Op>
__device__ __forceinline__ T scan_exclusive(T v, Op op) { return xlane::scan_exclusive(v, op); }

__device__ __forceinline__ float scan_inclusive_sum(__half v) { return scan_inclusive_sum(__half2float(v)); }
__device__ __forceinline__ float scan_inclusive_max(__half v) { return scan_inclusive_max(__half2float(v)); }
__device__ __forceinline__ float scan_inclusive_min(__half v) { return scan_inclusive_min(__half2float(v)); }
__device__ __forceinline__ float scan_exclusive_sum(__half v) { return scan_exclusive_sum(__half2float(v)); }
__device__ __forceinline__ float scan_inclusive_sum(__hip_bfloat16 v) { return scan_inclusive_sum(__bfloat162float(v)); }
__device__ __forceinline__ float scan_inclusive_max(__hip_bfloat16 v) { return scan_inclusive_max(__bfloat162float(v)); }
__device__ __forceinline__ float scan_inclusive_min(__hip_bfloat16 v) { return scan_inclusive_min(__bfloat162float(v)); }
__device__ __forceinline__ float scan_exclusive_sum(__hip_bfloat16 v) { return scan_exclusive_sum(__bfloat162float(v)); }
__device__ __forceinline__ float scan_inclusive_sum(hip_bfloat16 v) { return scan_inclusive_sum(float(v)); }
__device__ __forceinline__ float scan_inclusive_max(hip_bfloat16 v) { return scan_inclusive_max(float(v)); }
__device__ __forceinline__ float scan_inclusive_min(hip_bfloat16 v) { return scan_inclusive_min(float(v)); }
__device__ __forceinline__ float scan_exclusive_sum(hip_bfloat16 v) { return scan_exclusive_sum(float(v)); }

}  // namespace dpp
}  // namespace wave
