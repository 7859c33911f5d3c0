#pragma once
// cdna3::ex — row softmax building blocks on the zero-LDS wave reductions (same API as the
// reference's cdna3-prims/examples/fused_softmax.hpp:26-48).
#include "../cdna3.hpp"

namespace cdna3 {
namespace ex {

// One-shot softmax of a 64-wide row held one score per lane; returns this lane's probability.
__device__ __forceinline__ float row_softmax_lane(float score) {
    const float m = wave::dpp::reduce_max_bcast(score);
    const float e = __expf(score - m);
    const float s = wave::dpp::reduce_sum_bcast(e);
    return (s > 0.f) ? (e / s) : 0.f;
}

// Online-softmax update for one 64-wide tile: updates (m_run, l_run), writes this lane's
// unnormalised probability to p_out and returns the factor for rescaling the accumulator.
__device__ __forceinline__ float online_softmax_step(float score, float& m_run, float& l_run, float& p_out) {
    const float rmax = wave::dpp::reduce_max_bcast(score);
    const float mnew = fmaxf(m_run, rmax);
    const float p = __expf(score - mnew);
    const float rsum = wave::dpp::reduce_sum_bcast(p);
    const float resc = __expf(m_run - mnew);
    m_run = mnew;
    l_run = resc * l_run + rsum;
    p_out = p;
    return resc;
}

}  // namespace ex
}  // namespace cdna3
