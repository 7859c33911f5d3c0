#pragma once
// cdna3/wave.hpp — facade re-export of the wave64 primitive library (same role as the
// reference's cdna3-prims/include/cdna3/wave.hpp:24-26): wave::dpp::* (zero-LDS reductions and
// scans, re-derived for gfx950) and the reference-compatible wave::* API.
#include "../wave_primitives/wave_primitives.hpp"
#include "../wave_primitives/wave_reduce_dpp.hpp"
#include "../wave_primitives/wave_scan_dpp.hpp"
