#pragma once
// Cross-lane building blocks for gfx950 (CDNA4), all on the VALU path: DPP lane
// routing inside a 16-lane row and the gfx950 v_permlane16_swap / v_permlane32_swap
// instructions across rows. None of them touches LDS (no ds_* instruction, no
// ds_bpermute), and none goes through an SGPR (no v_readlane).
//
// Lane routing, checked lane by lane on an MI355X with an in-bounds probe:
//   quad_perm [1,0,3,2] (0xB1)   lane i <- lane i^1
//   quad_perm [2,3,0,1] (0x4E)   lane i <- lane i^2
//   row_half_mirror     (0x141)  lane i <- lane 7-i inside each 8-lane half row
//   row_mirror          (0x140)  lane i <- lane 15-i inside each 16-lane row
//   row_shr:n           (0x110+n) lane i <- lane i-n inside its row, else `old`
//   row_newbcast:15     (0x15F)  every lane <- lane 15 of its own row
//   permlane16_swap(a,b) -> {a', b'}: rows (0,1) and (2,3) are pairs;
//        a' = a with its odd rows replaced by b's even rows,
//        b' = b with its even rows replaced by a's odd rows.
//        With a == b == x: a' = x of the pair's even row, b' = x of the odd row.
//   permlane32_swap(a,b) -> {a', b'}: same, with 32-lane halves in place of rows.
//
// 64-bit values are moved as two 32-bit halves; the combine happens in 64 bits.
#include "config.hpp"
#include <type_traits>
#include <limits>

namespace wave {
namespace xlane {

enum : int {
    kQuadXor1      = 0xB1,
    kQuadXor2      = 0x4E,
    kRowHalfMirror = 0x141,
    kRowMirror     = 0x140,
    kRowShr1       = 0x111,
    kRowShr2       = 0x112,
    kRowShr4       = 0x114,
    kRowShr8       = 0x118,
    kRowNewBcast15 = 0x15F,
};

template <typename T>
__device__ __forceinline__ uint32_t lo32(T v) {
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(uint32_t, v);
    else return (uint32_t)__builtin_bit_cast(uint64_t, v);
}
template <typename T>
__device__ __forceinline__ uint32_t hi32(T v) {
    static_assert(sizeof(T) == 8, "hi32: 64-bit types only");
    return (uint32_t)(__builtin_bit_cast(uint64_t, v) >> 32);
}
template <typename T>
__device__ __forceinline__ T join(uint32_t lo, uint32_t hi) {
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, lo);
    else return __builtin_bit_cast(T, ((uint64_t)hi << 32) | (uint64_t)lo);
}

// DPP move: lanes whose source is outside the row read `old` (bound_ctrl off).
template <int Ctrl, typename T>
__device__ __forceinline__ T dpp(T old, T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "dpp: 32- or 64-bit types");
    if constexpr (sizeof(T) == 4) {
        return join<T>(__builtin_amdgcn_update_dpp(lo32(old), lo32(v), Ctrl, 0xf, 0xf, false), 0);
    } else {
        uint32_t lo = __builtin_amdgcn_update_dpp(lo32(old), lo32(v), Ctrl, 0xf, 0xf, false);
        uint32_t hi = __builtin_amdgcn_update_dpp(hi32(old), hi32(v), Ctrl, 0xf, 0xf, false);
        return join<T>(lo, hi);
    }
}

// DPP move for patterns with a source lane for every lane (quad_perm, mirrors,
// newbcast): `old` is never read. bound_ctrl is set so the compiler can fuse the move
// into the consuming VALU op (v_add_f32_dpp, v_max_f32_dpp, ...).
template <int Ctrl, typename T>
__device__ __forceinline__ T dpp_full(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "dpp_full: 32- or 64-bit types");
    if constexpr (sizeof(T) == 4) {
        return join<T>(__builtin_amdgcn_update_dpp(0u, lo32(v), Ctrl, 0xf, 0xf, true), 0);
    } else {
        uint32_t lo = __builtin_amdgcn_update_dpp(0u, lo32(v), Ctrl, 0xf, 0xf, true);
        uint32_t hi = __builtin_amdgcn_update_dpp(0u, hi32(v), Ctrl, 0xf, 0xf, true);
        return join<T>(lo, hi);
    }
}

// DPP move whose out-of-row lanes read zero (bound_ctrl): the identity of a sum, and a form
// the compiler fuses into v_add_*_dpp.
template <int Ctrl, typename T>
__device__ __forceinline__ T dpp_zero(T v) {
    return dpp_full<Ctrl>(v);
}

// Pair-of-rows exchange. Returns the pair's even-row value in `ev`, odd-row in `od`.
template <typename T>
__device__ __forceinline__ void rows_pair(T x, T& ev, T& od) {
    if constexpr (sizeof(T) == 4) {
        auto r = __builtin_amdgcn_permlane16_swap(lo32(x), lo32(x), false, false);
        ev = join<T>(r[0], 0);
        od = join<T>(r[1], 0);
    } else {
        auto rl = __builtin_amdgcn_permlane16_swap(lo32(x), lo32(x), false, false);
        auto rh = __builtin_amdgcn_permlane16_swap(hi32(x), hi32(x), false, false);
        ev = join<T>(rl[0], rh[0]);
        od = join<T>(rl[1], rh[1]);
    }
}

// Half-wave exchange. Returns the lower-half value in `lo`, upper-half in `up`.
template <typename T>
__device__ __forceinline__ void halves(T x, T& lo, T& up) {
    if constexpr (sizeof(T) == 4) {
        auto r = __builtin_amdgcn_permlane32_swap(lo32(x), lo32(x), false, false);
        lo = join<T>(r[0], 0);
        up = join<T>(r[1], 0);
    } else {
        auto rl = __builtin_amdgcn_permlane32_swap(lo32(x), lo32(x), false, false);
        auto rh = __builtin_amdgcn_permlane32_swap(hi32(x), hi32(x), false, false);
        lo = join<T>(rl[0], rh[0]);
        up = join<T>(rl[1], rh[1]);
    }
}

__device__ __forceinline__ unsigned lane() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// ---- combine operators ------------------------------------------------------
// Integer sums wrap in two's complement (computed in the unsigned type), so a
// device reduction is bit-identical to any other order of the same additions.
struct Sum {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
        if constexpr (std::is_integral<T>::value) {
            using U = typename std::make_unsigned<T>::type;
            return (T)((U)a + (U)b);
        } else {
            return a + b;
        }
    }
    template <typename T> __device__ __forceinline__ static T identity() { return T(0); }
};
struct Max {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a > b ? a : b; }
    template <typename T> __device__ __forceinline__ static T identity() { return std::numeric_limits<T>::lowest(); }
};
struct Min {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? a : b; }
    template <typename T> __device__ __forceinline__ static T identity() { return std::numeric_limits<T>::max(); }
};
struct And {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a & b; }
    template <typename T> __device__ __forceinline__ static T identity() { return (T)~T(0); }
};
struct Or {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a | b; }
    template <typename T> __device__ __forceinline__ static T identity() { return T(0); }
};

// ---- all-lanes reduction ----------------------------------------------------
// Butterfly: xor-1 and xor-2 inside quads, half-row mirror, row mirror (row total on
// all 16 lanes), then the row-pair swap and the half-wave swap. Every step combines
// two symmetric partners with the same operand order on both sides, so all 64 lanes
// end with a bit-identical value, also for floating-point sums.
template <typename Op, typename T>
__device__ __forceinline__ T allreduce(T v, Op op) {
    v = op(v, dpp_full<kQuadXor1>(v));
    v = op(v, dpp_full<kQuadXor2>(v));
    v = op(v, dpp_full<kRowHalfMirror>(v));
    v = op(v, dpp_full<kRowMirror>(v));
    T ev, od;
    rows_pair(v, ev, od);
    v = op(ev, od);
    T lo, up;
    halves(v, lo, up);
    return op(lo, up);
}

// Reduction over the 16 lanes of each row, result on all lanes of that row.
template <typename Op, typename T>
__device__ __forceinline__ T row_allreduce(T v, Op op) {
    v = op(v, dpp_full<kQuadXor1>(v));
    v = op(v, dpp_full<kQuadXor2>(v));
    v = op(v, dpp_full<kRowHalfMirror>(v));
    return op(v, dpp_full<kRowMirror>(v));
}

// Reduction across the four rows for each lane position (lanes i, i+16, i+32, i+48),
// result on all four lanes. Used where a value is spread over rows, e.g. the four
// lane groups that hold one query row of an MFMA 16x16 output tile.
template <typename Op, typename T>
__device__ __forceinline__ T cross_row_allreduce(T v, Op op) {
    T ev, od;
    rows_pair(v, ev, od);
    v = op(ev, od);
    T lo, up;
    halves(v, lo, up);
    return op(lo, up);
}

// Value of lane 63 on every lane: row_newbcast:15 spreads each row's lane 15, the
// row-pair swap picks row 3 in the upper pair, the half swap carries it down.
template <typename T>
__device__ __forceinline__ T lane63(T v) {
    const T r = dpp_full<kRowNewBcast15>(v);
    T ev, od;
    rows_pair(r, ev, od);
    T lo, up;
    halves(od, lo, up);
    return up;
}

// ---- inclusive scan ---------------------------------------------------------
// In-row Hillis-Steele over row_shr 1/2/4/8 (lanes without a source read the
// identity), then the carry from earlier rows: row_newbcast:15 gives each lane its
// own row total t_r; the row-pair swap yields t_even/t_odd of the pair; the half-wave
// swap yields the lower half's pair total. carry(row) = {0, t0, t0+t1, (t0+t1)+t2}.
// Returns the inclusive value and, through `carry`, the total of all earlier rows.
template <typename Op, typename T>
__device__ __forceinline__ T scan_with_carry(T v, Op op, T& carry) {
    const T id = Op::template identity<T>();
    if constexpr (std::is_same<Op, Sum>::value) {
        // Sum: out-of-row lanes read 0 through bound_ctrl, which fuses into v_add_*_dpp.
        v = op(v, dpp_zero<kRowShr1>(v));
        v = op(v, dpp_zero<kRowShr2>(v));
        v = op(v, dpp_zero<kRowShr4>(v));
        v = op(v, dpp_zero<kRowShr8>(v));
    } else {
        v = op(v, dpp<kRowShr1>(id, v));
        v = op(v, dpp<kRowShr2>(id, v));
        v = op(v, dpp<kRowShr4>(id, v));
        v = op(v, dpp<kRowShr8>(id, v));
    }
    const T rt = dpp_full<kRowNewBcast15>(v);   // this row's total on every lane
    T ev, od;
    rows_pair(rt, ev, od);                       // pair's even / odd row totals
    const T pair_total = op(ev, od);
    T lo, up;
    halves(pair_total, lo, up);                  // lower pair total on every lane
    const unsigned L = lane();
    const T pair_carry = (L & 16u) ? ev : id;    // odd row: even partner's total
    const T half_carry = (L & 32u) ? lo : id;    // upper half: lower pair's total
    carry = op(half_carry, pair_carry);
    return (L >= 16u) ? op(carry, v) : v;
}

template <typename Op, typename T>
__device__ __forceinline__ T scan_inclusive(T v, Op op) {
    T carry;
    return scan_with_carry(v, op, carry);
}

// Exclusive scan: row_shr:1 of the inclusive result; the lanes that start a row
// (0, 16, 32, 48) have no in-row source and take `old`, which is each lane's own
// carry (the identity on lane 0). That carry is bit-identical to the inclusive value
// of the previous row's last lane, because both are formed by the same operations.
template <typename Op, typename T>
__device__ __forceinline__ T scan_exclusive(T v, Op op) {
    T carry;
    const T inc = scan_with_carry(v, op, carry);
    return dpp<kRowShr1>(carry, inc);
}

}  // namespace xlane
}  // namespace wave
