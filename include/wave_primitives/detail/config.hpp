#pragma once
// Wave-primitive configuration for gfx950 (CDNA4), wave64 only.
//
// The reference library selected between an AMD DPP path and an NVIDIA __shfl path
// with WP_AMD / WP_NVIDIA (research/wave-primitives/include/wave_primitives/detail/
// config.hpp:4-24). This build targets one architecture, so both macros are fixed and
// kept only so existing `#if WP_AMD` blocks in caller code keep compiling.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WP_AMD 1
#define WP_NVIDIA 0

// 64-lane wave mask, as in the reference (config.hpp:16-24).
using wp_mask_t = unsigned long long;
#define WP_FULL_MASK 0xffffffffffffffffULL

namespace wave {
// Wave width of every gfx9-family compute wave this library is compiled for.
static constexpr int kWaveSize = 64;
}  // namespace wave
