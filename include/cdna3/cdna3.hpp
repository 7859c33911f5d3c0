#pragma once
// cdna3/cdna3.hpp — umbrella header (reference: cdna3-prims/include/cdna3/cdna3.hpp):
//   wave::dpp::reduce_* / scan_*   zero-LDS wave64 reductions and scans (gfx950 DPP + permlane)
//   dme::copy_*                    asynchronous HBM -> LDS copies (4- and 16-byte lanes)
//   cdna3::mfma::*                 16x16x16 f16 matrix-core accessors (reference API)
//   cdna4::mfma::*                 16x16x32 / 32x32x16 f16 and bf16 accessors (CDNA4)
// The attention launchers are in <cdna3/attention.hpp>; they need libcdna4_attn.so at link time.
#include "wave.hpp"
#include "dme.hpp"
#include "mfma.hpp"

namespace cdna3 {
// Library version. 1.0: gfx950 rebuild of the 0.2 API.
static constexpr int VERSION_MAJOR = 1;
static constexpr int VERSION_MINOR = 0;
}  // namespace cdna3
