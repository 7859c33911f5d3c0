#pragma once
// Umbrella header of the wave64 primitive library (gfx950), same include path and
// contents as the reference's (research/wave-primitives/include/wave_primitives/
// wave_primitives.hpp): shuffles, votes, reductions, scans. The zero-LDS
// wave::dpp:: forms are in wave_reduce_dpp.hpp and wave_scan_dpp.hpp.
#include "wave_shuffle.hpp"
#include "wave_ballot.hpp"
#include "wave_reduce.hpp"
#include "wave_scan.hpp"
