#pragma once
// wave:: vote operations, wave64 (64-bit masks).
//
// Names and semantics follow the reference (research/wave-primitives/include/
// wave_primitives/wave_ballot.hpp:26-82): activemask, ballot, any, all, popcount,
// lane_mask_lt, lane_mask_le. Note lane_mask_le keeps the reference's definition,
// which returns only the lane's own bit (wave_ballot.hpp:78-80).
#include "detail/config.hpp"
#include "wave_shuffle.hpp"

namespace wave {

__device__ __forceinline__ wp_mask_t activemask() { return (wp_mask_t)__builtin_amdgcn_read_exec(); }
__device__ __forceinline__ wp_mask_t ballot(int predicate) { return (wp_mask_t)__ballot(predicate); }
__device__ __forceinline__ int any(int predicate) { return ballot(predicate) != 0ull; }
__device__ __forceinline__ int all(int predicate) { return ballot(predicate) == activemask(); }
__device__ __forceinline__ int popcount(int predicate) { return __builtin_popcountll(ballot(predicate)); }
__device__ __forceinline__ wp_mask_t lane_mask_lt() {
    const unsigned l = lane_id();
    return (l == 0) ? 0ull : ((1ull << l) - 1ull);
}
__device__ __forceinline__ wp_mask_t lane_mask_le() { return 1ull << lane_id(); }

}  // namespace wave
