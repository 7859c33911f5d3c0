// Host replay of the device-wide scan's address arithmetic (test only, plain C++).
//
// Uses the same constexpr functions the kernels and their launcher use
// (amd-incstinct-labs_amd/csrc/scan_layout.hpp) and walks, for each element type, tile size and
// input size given, every vector / element load and store of every lane of every tile (tiles in
// groups of scan_waves(input bytes) waves, the last group's extra waves touching nothing), every slot word a
// tile group publishes or reads during its look-back, the header words and the tail's reads, checking each against the sizes of the input, output and workspace buffers (the
// workspace sized as cdna3_scan_workspace_size sizes it). Both the aligned (16-byte vector) and the
// misaligned (element-wise, half-size tiles) paths are replayed.
// Usage: scan_layout_check [--plant] U n [n ...]   (U = vectors per lane of the aligned path for 4- and
// 8-byte inputs, twice that for 16-bit ones, half of it on the misaligned path: scan_layout::scan_u;
// prints "ok <checks>" or the first violation and exits 1). --plant replays a deliberately wrong
// guard for the last tile (one vector more per lane than the tile holds) to show that the replay
// catches such an overrun.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "scan_layout.hpp"

namespace sl = cdna4::scan_layout;

struct Type {
    const char* name;
    int in_bytes, out_bytes;   // element sizes of input and output
    int VEC;                   // elements per vector load (ScanElem<DT>::VEC)
    int NW;                    // 64-bit words per tile slot (sizeof(Acc) / 4)
};

// f32, f64, i32, i64: 16-byte vectors; f16 / bf16: 8-byte loads of four values, fp32 output.
static const Type kTypes[] = {
    {"f32", 4, 4, 4, 1}, {"f64", 8, 8, 2, 2}, {"i32", 4, 4, 4, 1}, {"i64", 8, 8, 2, 2}, {"f16", 2, 4, 4, 1},
    {"bf16", 2, 4, 4, 1},
};

static unsigned long long g_checks = 0;
static bool g_plant = false;

#define CHECK(cond, ...)                                                  \
    do {                                                                  \
        ++g_checks;                                                       \
        if (!(cond)) {                                                    \
            printf("violation: " __VA_ARGS__);                            \
            printf("\n");                                                 \
            exit(1);                                                      \
        }                                                                 \
    } while (0)

// One call: n elements, input `in_off` bytes past a 16-byte boundary (0: the aligned path).
static void replay(const Type& T, int U, size_t n, size_t in_off) {
    const bool vec = in_off == 0;
    const int VEC = T.VEC;
    const int u = sl::scan_u(T.in_bytes, vec, U);
    // workspace as sized by cdna3_scan_workspace_size: the misaligned (smaller) tiles' count
    const size_t ws_tiles = sl::tiles_for(n, VEC, sl::scan_u(T.in_bytes, false, U));
    const size_t ws = sl::ws_bytes(ws_tiles);
    const size_t n_main = sl::main_elems(n, vec, VEC);
    const size_t ntiles = sl::tiles_for(n_main, VEC, u);
    const size_t TILE = sl::tile_elems(VEC, u);
    const size_t in_end = in_off + n * (size_t)T.in_bytes;   // bytes of the input buffer from its 16-byte base
    const size_t out_end = n * (size_t)T.out_bytes;
    const int waves = sl::scan_waves(T.in_bytes);
    const size_t ngroups = sl::groups_for(ntiles, waves);
    const size_t slot_bytes = ngroups * (size_t)T.NW * 8;
    CHECK(ngroups <= ws_tiles, "%s U%d n%zu: %zu groups, workspace sized for %zu", T.name, U, n, ngroups, ws_tiles);
    CHECK(sl::agg_offset() >= 4 && sl::agg_offset() + slot_bytes <= sl::pre_offset(ngroups), "%s n%zu agg", T.name, n);
    CHECK(sl::pre_offset(ngroups) + slot_bytes <= ws, "%s n%zu pre", T.name, n);
    // header: the error and epoch words (two u32) before the agg array
    CHECK(8 <= sl::agg_offset() && sl::agg_offset() <= ws, "%s n%zu header", T.name, n);
    // every wave of every group maps to one tile; exactly the tiles below ntiles are live
    size_t live_tiles = 0;
    for (size_t g = 0; g < ngroups; ++g)
        for (unsigned wv = 0; wv < (unsigned)waves; ++wv)
            if (sl::group_tile(g, wv, waves) < ntiles) ++live_tiles;
    CHECK(live_tiles == ntiles, "%s n%zu: groups cover %zu of %zu tiles", T.name, n, live_tiles, ntiles);
    for (size_t t = 0; t < ntiles; ++t) {
        const size_t base = sl::tile_base(t, TILE);
        CHECK(base < n_main, "%s n%zu tile %zu base %zu", T.name, n, t, base);
        const bool full = vec && sl::tile_full(base, TILE, n_main);
        const uint32_t rem = sl::tile_rem(base, TILE, n_main);
        CHECK(rem >= 1 && base + rem <= n_main, "%s n%zu tile %zu rem", T.name, n, t);
        for (unsigned lane = 0; lane < 64; ++lane) {
            for (int j = 0; j < u; ++j) {
                if (vec) {
                    const bool live = g_plant ? (full || sl::vec_in_tile(j, lane) <= rem / (uint32_t)VEC)
                                              : sl::vec_live(full, j, lane, rem, VEC);
                    if (!live) continue;
                    const size_t e0 = base + (size_t)sl::vec_in_tile(j, lane) * VEC;   // first element
                    CHECK(e0 % VEC == 0 && e0 + VEC <= n_main, "%s n%zu tile %zu lane %u j %d: e0 %zu", T.name, n, t,
                          lane, j, e0);
                    CHECK(e0 * T.in_bytes + (size_t)VEC * T.in_bytes <= in_end, "%s load past input", T.name);
                    CHECK((e0 * T.in_bytes) % ((size_t)VEC * T.in_bytes) == 0, "%s load misaligned", T.name);
                    CHECK(e0 * T.out_bytes + (size_t)VEC * T.out_bytes <= out_end, "%s store past output", T.name);
                    CHECK((e0 * T.out_bytes) % 16 == 0, "%s store misaligned", T.name);
                } else {
                    for (int e = 0; e < VEC; ++e) {
                        const uint32_t i = sl::elem_in_tile(j, lane, e, VEC);
                        if (i >= rem) continue;
                        CHECK(base + i < n_main, "%s n%zu tile %zu: element %zu", T.name, n, t, base + i);
                        CHECK(in_off + (base + i + 1) * T.in_bytes <= in_end, "%s element load past input", T.name);
                        CHECK((base + i + 1) * T.out_bytes <= out_end, "%s element store past output", T.name);
                    }
                }
            }
        }
    }
    for (size_t t = 0; t < ngroups; ++t) {
        // the group's exchange line: its waves' tile totals and the group prefix, 8 bytes each at most
        const size_t x0 = sl::xchg_offset(ngroups) + t * sl::kXchgStride;
        CHECK(x0 >= sl::pre_offset(ngroups) + slot_bytes && x0 % 128 == 0, "%s n%zu exchange line %zu", T.name, n, t);
        CHECK(x0 + (size_t)(waves + 1) * 8 <= ws && (waves + 1) * 8 <= (int)sl::kXchgStride,
              "%s n%zu exchange line %zu past the workspace or its line", T.name, n, t);
        // publish: lanes 0 .. NW-1 of wave 0 write the words of group t's slot in both arrays
        for (unsigned w = 0; w < (unsigned)T.NW; ++w)
            CHECK((sl::slot_word(t, T.NW, w) + 1) * 8 <= slot_bytes, "%s n%zu publish group %zu", T.name, n, t);
        // look-back: window positions pos = t - 1, t - 65, ...; lane l reads group pos - l when >= 0
        for (long long pos = (long long)t - 1; pos >= 0; pos -= 64)
            for (unsigned lane = 0; lane < 64; ++lane) {
                const long long r = pos - (long long)lane;
                if (r < 0) continue;
                CHECK(r < (long long)t, "%s look-back reads a later group", T.name);
                for (unsigned w = 0; w < (unsigned)T.NW; ++w)
                    CHECK((sl::slot_word((size_t)r, T.NW, w) + 1) * 8 <= slot_bytes, "%s n%zu read group %lld", T.name,
                          n, r);
            }
    }
    // the one-wave tail of an aligned call: the last tile's prefix, then elements n_main .. n-1
    if (n_main < n) {
        CHECK(vec, "%s tail on the misaligned path", T.name);
        if (ngroups > 0) CHECK((sl::slot_word(ngroups - 1, T.NW, T.NW - 1) + 1) * 8 <= slot_bytes, "%s tail slot", T.name);
        CHECK(n - n_main < (size_t)VEC, "%s tail longer than a vector", T.name);
        CHECK(in_off + n * T.in_bytes <= in_end && n * T.out_bytes <= out_end, "%s tail", T.name);
    }
}

int main(int argc, char** argv) {
    int a0 = 1;
    if (argc > 1 && strcmp(argv[1], "--plant") == 0) {
        g_plant = true;
        a0 = 2;
    }
    if (argc < a0 + 2) return 2;
    const int U = atoi(argv[a0]);
    if (U < 2 || U % 2) return 2;
    for (int a = a0 + 1; a < argc; ++a) {
        const size_t n = strtoull(argv[a], nullptr, 10);
        for (const Type& T : kTypes) {
            replay(T, U, n, 0);
            replay(T, U, n, (size_t)T.in_bytes);   // one element in: the element-wise path
        }
    }
    printf("ok %llu\n", g_checks);
    return 0;
}
