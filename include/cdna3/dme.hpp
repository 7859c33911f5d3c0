#pragma once
// cdna3/dme.hpp — facade re-export of the asynchronous HBM -> LDS copy helpers (reference:
// cdna3-prims/include/cdna3/dme.hpp). gfx950 adds 16-byte lanes (dme::copy16, copy_tile_16B).
#include "../dme/dme_copy.hpp"
#include "../dme/tensor_prefetch.hpp"
