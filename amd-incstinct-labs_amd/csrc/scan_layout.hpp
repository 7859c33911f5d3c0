// Index and workspace arithmetic of the device-wide scan (reduce_scan.hip), as constexpr functions
// shared by the kernels, their launcher and a host-side replay (tests/native/scan_layout_check.cpp)
// that walks every load, store and tile-slot address of every tile for given sizes and checks it
// against the buffer and workspace sizes. Plain C++: clang compiles constexpr functions for host
// and device alike.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace cdna4 {
namespace scan_layout {

constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// A tile is 64 lanes x U vectors of VEC elements. U on the aligned path: kScanU for 4- and 8-byte
// inputs, twice that for 16-bit inputs (held packed, 8 bytes per vector); on the misaligned
// (element-wise) path half of kScanU.
constexpr int kScanU = 32;
constexpr int scan_u(int in_bytes, bool vec, int base = kScanU) { return vec ? (in_bytes == 2 ? 2 * base : base) : base / 2; }
constexpr size_t tile_elems(int vec, int u) { return (size_t)64 * vec * u; }
constexpr size_t tiles_for(size_t n, int vec, int u) { return (n + tile_elems(vec, u) - 1) / tile_elems(vec, u); }

// Workspace for `nslots` look-back slots (one per tile group): [error and epoch words, padded to 256 B]
// [agg slots: align256(nslots * 16)][pre slots: align256(nslots * 16)][exchange lines:
// nslots * kXchgStride], two 64-bit words per slot and array (one used by 32-bit values), and per
// group one 128-byte line in which its waves leave their tile totals and wave 0 the group's prefix
// (W + 1 values of at most 8 bytes, W the group's waves). The library sizes it by the misaligned
// path's tile count, which bounds the group count of either path.
constexpr size_t kXchgStride = 128;
constexpr size_t ws_bytes(size_t ntiles) { return 256 + 2 * align256(ntiles * 16) + align256(ntiles * kXchgStride); }
constexpr size_t agg_offset() { return 256; }
constexpr size_t pre_offset(size_t ntiles) { return 256 + align256(ntiles * 16); }
constexpr size_t xchg_offset(size_t ntiles) { return pre_offset(ntiles) + align256(ntiles * 16); }

// Aligned calls scan whole VEC-element vectors in the tiles and the last n % VEC elements in a
// one-wave tail; misaligned calls scan everything element by element.
constexpr size_t main_elems(size_t n, bool vec, int VEC) { return vec ? n - n % (size_t)VEC : n; }

// Tile t starts at element t * TILE; the elements it covers (TILE, or fewer for the last tile).
constexpr size_t tile_base(size_t tile, size_t TILE) { return tile * TILE; }
constexpr bool tile_full(size_t base, size_t TILE, size_t n) { return base + TILE <= n; }
constexpr uint32_t tile_rem(size_t base, size_t TILE, size_t n) {
    return base + TILE <= n ? (uint32_t)TILE : (uint32_t)(n - base);
}
// Vector j of lane `lane` in a tile: its index among the tile's vectors, and the guard of the last
// (partial) tile: the vector is read and written only when it lies wholly inside the tile.
constexpr uint32_t vec_in_tile(int j, unsigned lane) { return (uint32_t)j * 64 + lane; }
constexpr bool vec_live(bool full, int j, unsigned lane, uint32_t rem, int VEC) {
    return full || vec_in_tile(j, lane) < rem / (uint32_t)VEC;
}
// Element e of vector j of a lane on the element-wise (misaligned) path, and its guard.
constexpr uint32_t elem_in_tile(int j, unsigned lane, int e, int VEC) { return vec_in_tile(j, lane) * (uint32_t)VEC + e; }

// Tiles run in workgroups of W waves, one tile per wave: wave w of workgroup g scans tile g W + w
// (waves past the last tile load and store nothing). The waves' totals meet in the workgroup, and
// the look-back state (a slot per published value) is per workgroup: a group publishes the total
// of its tiles and then its inclusive prefix. W = 4, and 8 for 8-byte inputs, whose tiles hold
// half the elements of 4-byte ones, so that twice as many look-backs would trail the stream (i64
// 2^26: 199.8 us with four waves, 187.3 with eight; f32 100.8 with four, 112.6 with eight, 109.7
// with two; f16 77.5 / 83.1 / 87.2).
constexpr int kScanWavesMax = 8;
constexpr int scan_waves(int in_bytes) { return in_bytes == 8 ? 8 : 4; }
static_assert((kScanWavesMax + 1) * 8 <= (int)kXchgStride, "a group's exchange values fit its line");
constexpr size_t groups_for(size_t ntiles, int waves) { return (ntiles + waves - 1) / waves; }
constexpr size_t group_tile(size_t group, unsigned wave, int waves) { return group * waves + wave; }

// 64-bit word w of group (slot) t's slot (NW words per slot).
constexpr size_t slot_word(size_t tile, int nw, unsigned w) { return tile * (size_t)nw + w; }

}  // namespace scan_layout
}  // namespace cdna4
