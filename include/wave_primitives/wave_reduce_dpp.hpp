#pragma once
// wave::dpp reductions for gfx950 (CDNA4), wave64, zero LDS instructions.
//
// Same names, argument and return types as the reference's wave::dpp reductions
// (research/wave-primitives/include/wave_primitives/wave_reduce_dpp.hpp:56-113):
//   reduce_sum / reduce_max / reduce_min        result on lane 63
//   reduce_sum_bcast / _max_bcast / _min_bcast  result on every lane
//   id_sum / id_max / id_min, SumOp / MaxOp / MinOp, dpp_reduce, dpp_move, bcast_lane63
//
// Unlike the reference's lane-63 chain (row_shr 1/2/4/8 + row_bcast15/31, then
// v_readlane for the broadcast), every reduction here is an all-lanes butterfly
// (see detail/xlane.hpp): the result is on lane 63 and on every other lane, with
// no SGPR round trip, so the _bcast forms cost nothing extra.
//
// New in this build: fp16 / bf16 inputs accumulate in fp32 and return float
// (reduce_sum(__half) -> float, ...).
#include "detail/xlane.hpp"
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <hip/hip_bfloat16.h>

namespace wave {
namespace dpp {

template <typename T> __device__ __forceinline__ T id_sum() { return T(0); }
template <typename T> __device__ __forceinline__ T id_max() { return std::numeric_limits<T>::lowest(); }
template <typename T> __device__ __forceinline__ T id_min() { return std::numeric_limits<T>::max(); }

using SumOp = xlane::Sum;
using MaxOp = xlane::Max;
using MinOp = xlane::Min;

// One DPP move with control code Ctrl (row/bank masks all on): lane i receives the Ctrl-selected
// lane's v, or old_val where that lane is outside the row (e.g. row_shr:1 = 0x111 gives each row's
// lane 0 old_val). 32- and 64-bit types (a 64-bit value moves as two 32-bit halves).
template <int Ctrl, typename T>
__device__ __forceinline__ T dpp_move(T v, T old_val) {
    return xlane::dpp<Ctrl>(old_val, v);
}

// Full-wave combine with an arbitrary associative, commutative functor. The identity
// argument is kept for signature compatibility; the butterfly never reads it.
template <typename T, typename Op>
__device__ __forceinline__ T dpp_reduce(T v, Op op, T /*identity*/) {
    return xlane::allreduce(v, op);
}

// Value of lane 63 on every lane, for arbitrary per-lane data (three VALU cross-lane
// steps, see xlane::lane63). The reductions in this header do not need it: their
// result is already on every lane.
template <typename T>
__device__ __forceinline__ T bcast_lane63(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "bcast_lane63: only 32/64-bit types");
    return xlane::lane63(v);
}

template <typename T> __device__ __forceinline__ T reduce_sum(T v) { return xlane::allreduce(v, SumOp{}); }
template <typename T> __device__ __forceinline__ T reduce_max(T v) { return xlane::allreduce(v, MaxOp{}); }
template <typename T> __device__ __forceinline__ T reduce_min(T v) { return xlane::allreduce(v, MinOp{}); }

template <typename T> __device__ __forceinline__ T reduce_sum_bcast(T v) { return reduce_sum(v); }
template <typename T> __device__ __forceinline__ T reduce_max_bcast(T v) { return reduce_max(v); }
template <typename T> __device__ __forceinline__ T reduce_min_bcast(T v) { return reduce_min(v); }

// fp16 / bf16 inputs: fp32 accumulation, fp32 result.
__device__ __forceinline__ float reduce_sum(__half v) { return reduce_sum(__half2float(v)); }
__device__ __forceinline__ float reduce_max(__half v) { return reduce_max(__half2float(v)); }
__device__ __forceinline__ float reduce_min(__half v) { return reduce_min(__half2float(v)); }
__device__ __forceinline__ float reduce_sum(__hip_bfloat16 v) { return reduce_sum(__bfloat162float(v)); }
__device__ __forceinline__ float reduce_max(__hip_bfloat16 v) { return reduce_max(__bfloat162float(v)); }
__device__ __forceinline__ float reduce_min(__hip_bfloat16 v) { return reduce_min(__bfloat162float(v)); }
__device__ __forceinline__ float reduce_sum_bcast(__half v) { return reduce_sum(v); }
__device__ __forceinline__ float reduce_max_bcast(__half v) { return reduce_max(v); }
__device__ __forceinline__ float reduce_min_bcast(__half v) { return reduce_min(v); }
__device__ __forceinline__ float reduce_sum_bcast(__hip_bfloat16 v) { return reduce_sum(v); }
__device__ __forceinline__ float reduce_max_bcast(__hip_bfloat16 v) { return reduce_max(v); }
__device__ __forceinline__ float reduce_min_bcast(__hip_bfloat16 v) { return reduce_min(v); }
__device__ __forceinline__ float reduce_sum(hip_bfloat16 v) { return reduce_sum(float(v)); }
__device__ __forceinline__ float reduce_max(hip_bfloat16 v) { return reduce_max(float(v)); }
__device__ __forceinline__ float reduce_min(hip_bfloat16 v) { return reduce_min(float(v)); }
__device__ __forceinline__ float reduce_sum_bcast(hip_bfloat16 v) { return reduce_sum(float(v)); }
__device__ __forceinline__ float reduce_max_bcast(hip_bfloat16 v) { return reduce_max(float(v)); }
__device__ __forceinline__ float reduce_min_bcast(hip_bfloat16 v) { return reduce_min(float(v)); }

}  // namespace dpp
}  // namespace wave
