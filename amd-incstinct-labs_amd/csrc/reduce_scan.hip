// Device-wide reduce and inclusive scan built on the wave64 DPP primitives (gfx950).
//
// The reference has these operations only at wave level (research/wave-primitives/
// include/wave_primitives/wave_reduce_dpp.hpp:106-113, wave_scan_dpp.hpp:70-87). Here
// they run over whole HBM arrays without a single LDS instruction:
//   reduce: stage 1 streams the input with 16-byte loads, each wave folds its share in
//           registers and combines its 64 lanes with the DPP/permlane butterfly, then
//           writes one partial; stage 2 (one wave) folds the partials.
//   scan:   one pass with decoupled look-back. Each wave scans a tile held in registers
//           (per-lane serial + wave scan per 64x16-byte chunk); the four waves of a
//           workgroup meet their tile totals in a line of the workspace, and the group
//           publishes its aggregate, reads its predecessor groups' aggregates / prefixes 64
//           at a time (one per lane) and writes the output. Every published word carries the
//           call's epoch, so words left by earlier calls read as "not ready" and the flags need
//           no clearing between calls. No LDS in either.
#include <type_traits>
#include "common.hpp"
#include <atomic>
#include <stdlib.h>
#include <time.h>
#include <unistd.h>
#include "scan_layout.hpp"
#include "wave_primitives/detail/xlane.hpp"

namespace cdna4 {
namespace {

using wave::xlane::allreduce;
using wave::xlane::scan_with_carry;
using wave::xlane::dpp;
using wave::xlane::kRowShr1;

// ---- element traits: 16-byte vector <-> accumulator values ------------------------
template <int DT> struct Elem;
template <> struct Elem<CDNA4_F32> {
    using In = float; using Acc = float; using Out = float; static constexpr int VEC = 4;
    __device__ static Acc load1(const In* p) { return *p; }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        // Element by value: clang folds __builtin_bit_cast of an ext-vector element lvalue
        // to element 0 (observed with ROCm 7.2 clang), so the element is copied first.
        o[0] = f32_from_bits(v[0]); o[1] = f32_from_bits(v[1]);
        o[2] = f32_from_bits(v[2]); o[3] = f32_from_bits(v[3]);
    }
};
template <> struct Elem<CDNA4_I32> {
    using In = int32_t; using Acc = int32_t; using Out = int32_t; static constexpr int VEC = 4;
    __device__ static Acc load1(const In* p) { return *p; }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        o[0] = (int32_t)v[0]; o[1] = (int32_t)v[1]; o[2] = (int32_t)v[2]; o[3] = (int32_t)v[3];
    }
};
template <> struct Elem<CDNA4_F64> {
    using In = double; using Acc = double; using Out = double; static constexpr int VEC = 2;
    __device__ static Acc load1(const In* p) { return *p; }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        o[0] = __builtin_bit_cast(double, ((uint64_t)v[1] << 32) | v[0]);
        o[1] = __builtin_bit_cast(double, ((uint64_t)v[3] << 32) | v[2]);
    }
};
template <> struct Elem<CDNA4_I64> {
    using In = int64_t; using Acc = int64_t; using Out = int64_t; static constexpr int VEC = 2;
    __device__ static Acc load1(const In* p) { return *p; }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        o[0] = (int64_t)(((uint64_t)v[1] << 32) | v[0]);
        o[1] = (int64_t)(((uint64_t)v[3] << 32) | v[2]);
    }
};
template <> struct Elem<CDNA4_F16> {
    using In = uint16_t; using Acc = float; using Out = float; static constexpr int VEC = 8;
    __device__ static Acc load1(const In* p) { return f16_bits_to_f32(*p); }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        const uint32_t w[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) { o[2 * i] = f16_bits_to_f32(w[i] & 0xffffu); o[2 * i + 1] = f16_bits_to_f32(w[i] >> 16); }
    }
};
template <> struct Elem<CDNA4_BF16> {
    using In = uint16_t; using Acc = float; using Out = float; static constexpr int VEC = 8;
    __device__ static Acc load1(const In* p) { return bf16_bits_to_f32(*p); }
    __device__ static void unpack(const u32x4& v, Acc (&o)[VEC]) {
        const uint32_t w[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) { o[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu); o[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16); }
    }
};

using OpSum = wave::xlane::Sum;
using OpMax = wave::xlane::Max;
using OpMin = wave::xlane::Min;

// ---- reduce -------------------------------------------------------------------------
constexpr int kReduceThreads = 256;          // 4 waves, no LDS: each wave writes a partial
constexpr int kReduceMaxBlocks = 2048;       // 8192 partials at most
// 16-byte loads in flight per lane. Each block reads kReduceThreads * 4 consecutive vectors per
// step (its four loads per lane 4 KiB apart), the steps strided over the grid: at 2^26 on the
// MI355X this ran f32 49.1 -> 42.8 us, f64 96.9 -> 81.0, bf16 26.0 -> 23.7 against four loads per
// lane spread a whole grid apart (8 MiB); eight loads per lane were no faster in either layout.
template <int DT>
constexpr int reduce_unroll() { return 4; }

// kVec: in_ is 16-byte aligned and read as vectors; the nhead (< one vector) elements at head_
// that precede it (a misaligned call's first elements) are folded in by the first threads.
template <int DT, class Op, bool kVec>
__global__ __launch_bounds__(kReduceThreads) void reduce_stage1(const void* __restrict__ in_, size_t n,
                                                                 void* __restrict__ part_,
                                                                 const void* __restrict__ head_, int nhead) {
    using E = Elem<DT>;
    using Acc = typename E::Acc;
    const typename E::In* in = (const typename E::In*)in_;
    Op op;
    const Acc id = Op::template identity<Acc>();
    constexpr int kReduceUnroll = reduce_unroll<DT>();
    Acc acc[kReduceUnroll];
#pragma unroll
    for (int u = 0; u < kReduceUnroll; ++u) acc[u] = id;
    const size_t nthr = (size_t)gridDim.x * kReduceThreads;
    const size_t tid = (size_t)blockIdx.x * kReduceThreads + threadIdx.x;
    size_t scalar_from = 0;
    if constexpr (kVec) {
        const u32x4* vin = (const u32x4*)in;
        const size_t nvec = n / E::VEC;
        constexpr size_t kGroup = (size_t)kReduceThreads * kReduceUnroll;   // vectors per block step
        const size_t full = nvec / kGroup * kGroup;
        for (size_t base = (size_t)blockIdx.x * kGroup; base < full; base += (size_t)gridDim.x * kGroup) {
            u32x4 v[kReduceUnroll];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                v[u] = __builtin_nontemporal_load(vin + base + u * kReduceThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u) {
                Acc x[E::VEC];
                E::unpack(v[u], x);
#pragma unroll
                for (int e = 0; e < E::VEC; ++e) acc[u] = op(acc[u], x[e]);
            }
        }
        for (size_t i = full + tid; i < nvec; i += nthr) {   // the last partial step
            Acc x[E::VEC];
            E::unpack(vin[i], x);
#pragma unroll
            for (int e = 0; e < E::VEC; ++e) acc[0] = op(acc[0], x[e]);
        }
        scalar_from = nvec * E::VEC;
    }
    for (size_t i = scalar_from + tid; i < n; i += nthr) acc[1] = op(acc[1], E::load1(in + i));
    if (tid < (size_t)nhead) acc[2] = op(acc[2], E::load1((const typename E::In*)head_ + tid));
    Acc a = acc[0];
#pragma unroll
    for (int u = 1; u < kReduceUnroll; ++u) a = op(a, acc[u]);
    a = allreduce(a, op);
    if ((threadIdx.x & 63u) == 0) ((Acc*)part_)[blockIdx.x * (kReduceThreads / 64) + threadIdx.x / 64] = a;
}

// Stage 2: 16 waves fold the partials (at most eight per thread, all eight loads issued before
// the first is used: one memory round trip), each wave writes one value after the partials, and
// after the workgroup barrier wave 0 folds those 16. Deterministic order, no LDS.
constexpr int kReduce2Threads = 1024;

template <int DT, class Op>
__global__ __launch_bounds__(kReduce2Threads) void reduce_stage2(void* __restrict__ part_, int count,
                                                                  void* __restrict__ out_) {
    using Acc = typename Elem<DT>::Acc;
    Acc* part = (Acc*)part_;
    Op op;
    const Acc id = Op::template identity<Acc>();
    static_assert(kReduceMaxBlocks * (kReduceThreads / 64) <= 8 * kReduce2Threads, "eight partials per thread");
    Acc v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = (int)threadIdx.x + u * kReduce2Threads;
        v[u] = i < count ? part[i] : id;
    }
    Acc a = op(op(op(v[0], v[1]), op(v[2], v[3])), op(op(v[4], v[5]), op(v[6], v[7])));
    a = allreduce(a, op);
    Acc* wave_vals = part + count;   // kReduce2Threads / 64 slots after the partials
    if ((threadIdx.x & 63u) == 0) wave_vals[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x < 64) {
        Acc v = (threadIdx.x < kReduce2Threads / 64) ? wave_vals[threadIdx.x] : id;
        v = allreduce(v, op);
        if (threadIdx.x == 0) *(Acc*)out_ = v;
    }
}

unsigned reduce_blocks(size_t n, int vec, int unroll) {
    const size_t per_block = (size_t)kReduceThreads * vec * unroll;
    size_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > kReduceMaxBlocks) b = kReduceMaxBlocks;
    return (unsigned)b;
}

template <int DT, class Op>
int reduce_launch(const void* in, size_t n, void* out, void* ws, hipStream_t s) {
    using E = Elem<DT>;
    constexpr size_t kEsz = sizeof(typename E::In);
    // A misaligned input (elements at their natural alignment) splits into the elements up to the
    // first 16-byte boundary, folded in by the first threads, and an aligned vector body.
    const uintptr_t addr = (uintptr_t)in;
    size_t head = 0;
    bool vec = addr % 16 == 0;
    if (!vec && addr % kEsz == 0) {
        head = (16 - addr % 16) / kEsz;
        vec = head < n;
        if (!vec) head = 0;
    }
    const unsigned blocks = reduce_blocks(n - head, E::VEC, reduce_unroll<DT>());
    if (vec)
        reduce_stage1<DT, Op, true><<<blocks, kReduceThreads, 0, s>>>((const char*)in + head * kEsz, n - head, ws, in,
                                                                       (int)head);
    else
        reduce_stage1<DT, Op, false><<<blocks, kReduceThreads, 0, s>>>(in, n, ws, nullptr, 0);
    reduce_stage2<DT, Op><<<1, kReduce2Threads, 0, s>>>(ws, (int)(blocks * (kReduceThreads / 64)), out);
    return launch_status();
}

// ---- scan (decoupled look-back over groups of four single-wave tiles) ------------------
// Scan layout per element type: 16-bit inputs load 8 bytes (4 values) per lane and vector, so
// each lane's fp32 output vector leaves as one 16-byte store and every store instruction writes
// 1 KiB of contiguous lines (16-byte loads of 8 values left each lane's 32-byte output as two
// stores 32 bytes apart, and the half-filled lines were written twice).
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
template <int DT> struct ScanElem : Elem<DT> {
    using Load = u32x4;
    // A vector of the op's identity, for the vectors past the end of the last tile.
    template <class Op> __device__ static Load ident() {
        using Acc = typename Elem<DT>::Acc;
        Acc a[Elem<DT>::VEC];
#pragma unroll
        for (int e = 0; e < Elem<DT>::VEC; ++e) a[e] = Op::template identity<Acc>();
        return __builtin_bit_cast(Load, a);
    }
};
template <int DT> struct ScanElem16 : Elem<DT> {
    using Load = u32x2;
    static constexpr int VEC = 4;
    // Four packed copies of the op's identity (0, -inf for max, +inf for min), for the vectors past
    // the end of the last tile.
    template <class Op> __device__ static Load ident() {
        constexpr bool kBf = DT == CDNA4_BF16;
        uint32_t h = 0u;
        if constexpr (std::is_same<Op, wave::xlane::Max>::value) h = kBf ? 0xFF80u : 0xFC00u;
        if constexpr (std::is_same<Op, wave::xlane::Min>::value) h = kBf ? 0x7F80u : 0x7C00u;
        return Load{h | (h << 16), h | (h << 16)};
    }
    __device__ static void unpack(const u32x2& v, float (&o)[4]) {
        const uint32_t w[2] = {v[0], v[1]};
        float x[8];
        u32x4 q = {w[0], w[1], 0u, 0u};
        Elem<DT>::unpack(q, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = x[i];
    }
};
template <> struct ScanElem<CDNA4_F16> : ScanElem16<CDNA4_F16> {};
template <> struct ScanElem<CDNA4_BF16> : ScanElem16<CDNA4_BF16> {};
// Tile = 64 lanes x U vectors per lane (scan_layout::scan_u). The look-back costs about the same
// per tile whatever its size, so tiles are as large as the register file allows at three waves per
// SIMD (~155 VGPRs with the tile held as loaded): 32 16-byte vectors for 32- and 64-bit inputs (24 /
// 36 / 40 ran 3-8 % slower), 64 8-byte vectors of four 16-bit values (48: 83 us, 64: 77 us, 80 at
// two waves: 87 us at 2^26; held as fp32 values they had fitted 32, 83 us).
template <int DT, bool kVec> constexpr int scan_u() { return scan_layout::scan_u((int)sizeof(typename Elem<DT>::In), kVec); }

// Per-group look-back state. A group publishes its aggregate into agg and, once known, its
// inclusive prefix into pre. Every 64-bit word carries a tag in its upper half and 32 value bits
// in its lower half; 64-bit values use two words (low, high half), and a reader accepts a slot only
// when all its words carry the tag it looks for, so a torn read is just "not ready". Value and tag
// travel in one atomic word, so relaxed device-scope atomics suffice: no release/acquire fences,
// which on this multi-XCD part would write back / invalidate the L2 on every publish and every
// poll. The tag is (epoch << 2) | kind (kind 1 = aggregate, 2 = prefix), the epoch a number the
// host draws per call (scan_epoch, never 0): a word left in the workspace by an earlier call
// carries another epoch and reads as "not ready", so the slots need no clearing between calls (an
// earlier build cleared them in a separate launch before every call). A zeroed workspace holds no
// valid tag at all; memory never written by a scan could, by chance, hold the exact 32-bit tag of
// the call in a word's upper half.
struct ScanState {
    uint64_t* agg;    // per group: NW words
    uint64_t* pre;    // per group: NW words
    uint32_t* error;  // set to the epoch when a look-back wait exceeds its bound
    uint32_t* epoch_word;   // the epoch of the last call on this workspace
    uint32_t epoch;
    uint64_t tag_agg, tag_pre;
    uint32_t spin_limit;   // sleeps a look-back waits for a predecessor before it gives up
    unsigned char* xchg;   // per group a 128-byte line: its waves' tile totals, then its prefix
};

constexpr uint32_t kSpinLimit = 1u << 22;

// The look-back's wait bound: kSpinLimit, or CDNA4_SCAN_SPIN_LIMIT from the environment when set
// (read on every call), so a test can force the timeout path from the host with a tiny bound while
// every kernel still runs to completion.
uint32_t scan_spin_limit() {
    const char* e = getenv("CDNA4_SCAN_SPIN_LIMIT");
    if (!e || !*e) return kSpinLimit;
    char* end = nullptr;
    const unsigned long v = strtoul(e, &end, 10);
    return (end && *end == 0 && v <= kSpinLimit) ? (uint32_t)v : kSpinLimit;
}
// Per-call epochs: 1 .. 2^30 - 2 in sequence from a start drawn per process (clock and pid), so
// that consecutive calls on a workspace, also from different processes, carry different tags.
uint32_t scan_epoch() {
    static std::atomic<uint32_t> next{(uint32_t)((uint64_t)time(nullptr) * 2654435761u) ^ ((uint32_t)getpid() << 16)};
    const uint32_t x = next.fetch_add(1, std::memory_order_relaxed);
    return x % 0x3FFFFFFEu + 1u;   // 1 .. 2^30 - 2: no tag is all ones
}

template <typename Acc> struct Words { static constexpr int NW = sizeof(Acc) / 4; };

template <typename Acc> __device__ __forceinline__ uint64_t to_bits(Acc v) {
    if constexpr (sizeof(Acc) == 4) return (uint64_t)__builtin_bit_cast(uint32_t, v);
    else return __builtin_bit_cast(uint64_t, v);
}
template <typename Acc> __device__ __forceinline__ Acc from_bits(uint64_t b) {
    if constexpr (sizeof(Acc) == 4) return __builtin_bit_cast(Acc, (uint32_t)b);
    else return __builtin_bit_cast(Acc, b);
}

__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lanes 0 .. NW-1 each write one word of tile t's slot.
template <typename Acc>
__device__ __forceinline__ void publish(uint64_t* slots, size_t t, Acc v, uint64_t tag) {
    constexpr int NW = Words<Acc>::NW;
    const unsigned lane = threadIdx.x;
    if (lane < (unsigned)NW) {
        const uint64_t bits = to_bits(v);
        const uint32_t half = (uint32_t)(lane == 0 ? bits : bits >> 32);
        st_word(slots + scan_layout::slot_word(t, NW, lane), (tag << 32) | half);
    }
}

// Reads tile t's slot: true and the value when every word carries the tag.
template <typename Acc>
__device__ __forceinline__ bool read_slot(const uint64_t* slots, long long t, uint64_t tag, Acc& v) {
    constexpr int NW = Words<Acc>::NW;
    const uint64_t w0 = ld_word(slots + scan_layout::slot_word((size_t)t, NW, 0));
    uint64_t bits = (uint32_t)w0;
    bool ok = (w0 >> 32) == tag;
    if constexpr (NW == 2) {
        const uint64_t w1 = ld_word(slots + scan_layout::slot_word((size_t)t, NW, 1));
        ok = ok && (w1 >> 32) == tag;
        bits |= (uint64_t)(uint32_t)w1 << 32;
    }
    v = from_bits<Acc>(bits);
    return ok;
}

// Combined value of all tiles before `tile`, on every lane. Lane i examines tile pos - i; the
// window moves back 64 tiles at a time until it contains a published prefix.
template <typename Acc, class Op>
__device__ Acc look_back(const ScanState& st, size_t tile, Op op) {
    const unsigned lane = threadIdx.x;
    const Acc id = Op::template identity<Acc>();
    Acc acc = id;
    long long pos = (long long)tile - 1;
    while (true) {
        const long long t = pos - (long long)lane;
        Acc v = id;
        uint32_t s = 2u;                 // lanes before tile 0 act as an (identity) prefix
        uint64_t mzero = 0, mpre = 0;
        for (uint32_t spin = 0;; ++spin) {
            if (t >= 0) {
                Acc pv, av;
                const bool p = read_slot<Acc>(st.pre, t, st.tag_pre, pv);
                const bool q = read_slot<Acc>(st.agg, t, st.tag_agg, av);
                s = p ? 2u : (q ? 1u : 0u);
                v = p ? pv : (q ? av : id);
            }
            mpre = __ballot(s == 2u);
            mzero = __ballot(s == 0u);
            const uint64_t below = mpre ? ((mpre & (~mpre + 1ull)) - 1ull) : ~0ull;  // lanes before first prefix
            if ((mzero & below) == 0ull) break;
            if (spin >= st.spin_limit) {
                if (lane == 0) __hip_atomic_store(st.error, st.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        const int first_pre = mpre ? __builtin_ctzll(mpre) : 64;
        if ((int)lane > first_pre || (t < 0 && (int)lane != first_pre)) v = id;
        acc = op(allreduce(v, op), acc);
        if (first_pre < 64) break;
        pos -= 64;
    }
    return acc;
}

// Wave w of workgroup g scans tile g W + w (scan_layout::group_tile, W = scan_waves: 4, or 8 for
// 8-byte inputs); the group runs one look-back for its W tiles. With one tile per single-wave
// workgroup the look-back was the bound: per-tile stamps showed a tile's loads arriving after
// 13 us and its look-back taking another 17 us (median, ~2 us per round trip of the device-scope
// slot words behind the stream), as prefixes trailed ~190 tiles behind the aggregates; four times
// fewer, larger look-back units took the f32 scan at 2^26 from 125 to 102 us (16-bit inputs 112 ->
// 83 us, 64-bit 253 -> 202 us, and 200 -> 187 us with eight-wave groups).
template <int DT> constexpr int scan_group_waves() { return scan_layout::scan_waves((int)sizeof(typename ScanElem<DT>::In)); }

template <int DT, class Op, bool kVec>
__global__ __launch_bounds__(64 * scan_group_waves<DT>()) void scan_tiles(const void* __restrict__ in_, size_t n,
                                                                          void* __restrict__ out_, ScanState st) {
    constexpr int kWaves = scan_group_waves<DT>();
    using E = ScanElem<DT>;
    using Acc = typename E::Acc;
    using Out = typename E::Out;
    constexpr int VEC = E::VEC;
    constexpr int U = scan_u<DT, kVec>();
    constexpr size_t TILE = scan_layout::tile_elems(VEC, U);
    const typename E::In* in = (const typename E::In*)in_;
    Out* out = (Out*)out_;
    Op op;
    const Acc id = Op::template identity<Acc>();
    const unsigned lane = threadIdx.x & 63u;
    const unsigned wave = threadIdx.x >> 6;
    const size_t group = blockIdx.x;
    const size_t tile = scan_layout::group_tile(group, wave, kWaves);
    const bool live = tile < (n + TILE - 1) / TILE;   // the last group's waves past the last tile: no memory access
    const size_t base = live ? scan_layout::tile_base(tile, TILE) : 0;
    // The group's exchange line in the workspace (global memory, no LDS): the waves' tile totals,
    // then the group's exclusive prefix. Written before and read after a workgroup barrier, as
    // reduce_stage2 meets its waves; each group owns a whole 128-byte line. In LDS the same
    // exchange measured no faster (102.5 against 103.2 us at f32 2^26).
    Acc* s_tot = (Acc*)(st.xchg + group * scan_layout::kXchgStride);
    Acc* s_excl = s_tot + kWaves;

    // Aligned calls (kVec): n counts the elements of whole VEC-element vectors only (the host
    // scans the remaining n % VEC elements in scan_tail). Every tile but the last is full and
    // takes a straight-line path of vector loads at fixed offsets from one base, all issued before
    // any arithmetic; the last tile guards each vector with a 32-bit tile-local index against the
    // uniform vector count. Misaligned calls go element by element.
    // 16- and 64-bit inputs on the aligned path (kRaw) keep the tile in registers as loaded (16-bit
    // values packed, two VGPRs per four) while only its total is formed, a fold per lane and one
    // over the wave, so the group's aggregate goes out before the tile's scan is computed, after the
    // look-back; past the end of the last tile the vectors hold the op's identity. Packed 16-bit
    // tiles hold twice the elements of scanned fp32 ones (f16 82 -> 76.5 us at 2^26, bf16 84 -> 78;
    // 64-bit 200 -> 198 us). 32-bit inputs hold the scanned values across the look-back instead,
    // so the stores follow it at once (held as loaded: f32 101.1 -> 101.8 us, i32 100.9 -> 103.0).
    const typename E::In* tin = in + base;
    const bool full = live && kVec && scan_layout::tile_full(base, TILE, n);
    const uint32_t rem = live ? scan_layout::tile_rem(base, TILE, n) : 0u;  // elements (0: none)
    // Local inclusive scan of one vector of VEC values per lane: within the lane, then across the
    // wave (DPP), carried on from `run`, the combined value of the tile's earlier vectors.
    auto scan_vec = [&](Acc (&x)[VEC], Acc& run) {
#pragma unroll
        for (int e = 1; e < VEC; ++e) x[e] = op(x[e - 1], x[e]);
        Acc carry;
        const Acc inc = scan_with_carry(x[VEC - 1], op, carry);
        const Acc exc = dpp<kRowShr1>(carry, inc);          // lane's exclusive within chunk
        const Acc pre = op(run, exc);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] = op(pre, x[e]);
        run = op(run, wave::xlane::lane63(inc));             // chunk total, on every lane
    };
    constexpr bool kRaw = kVec && sizeof(typename E::In) != 4;
    typename E::Load r[kRaw ? U : 1];   // kRaw: the tile as loaded
    Acc v[kRaw ? 1 : U][VEC];           // otherwise: the tile's scanned values
    Acc run = id;                       // the tile's total, on every lane
    if constexpr (kRaw) {
        const typename E::Load* src = (const typename E::Load*)tin + lane;
        if (full) {
#pragma unroll
            for (int j = 0; j < U; ++j) r[j] = __builtin_nontemporal_load(src + j * 64);
            __builtin_amdgcn_sched_barrier(0);
        } else {
#pragma unroll
            for (int j = 0; j < U; ++j)
                r[j] = scan_layout::vec_live(false, j, lane, rem, VEC) ? __builtin_nontemporal_load(src + j * 64)
                                                                      : E::template ident<Op>();
        }
        // For a float sum this total can differ from the last value of the scan after the look-back
        // by the rounding of the tile's total (a different order), which the next tiles then carry.
        Acc part[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) part[e] = id;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            Acc x[VEC];
            E::unpack(r[j], x);
#pragma unroll
            for (int e = 0; e < VEC; ++e) part[e] = op(part[e], x[e]);
        }
#pragma unroll
        for (int e = 1; e < VEC; ++e) part[0] = op(part[0], part[e]);
        run = allreduce(part[0], op);
        // The loaded tile, not this fold's values, is what stays live across the look-back.
#pragma unroll
        for (int j = 0; j < U; ++j) asm volatile("" : "+v"(r[j]));
    } else {
        if constexpr (kVec) {
            const typename E::Load* src = (const typename E::Load*)tin + lane;
            if (full) {
#pragma unroll
                for (int j = 0; j < U; ++j) E::unpack(__builtin_nontemporal_load(src + j * 64), v[j]);
                __builtin_amdgcn_sched_barrier(0);
            } else {
#pragma unroll
                for (int j = 0; j < U; ++j) {
                    if (scan_layout::vec_live(false, j, lane, rem, VEC)) {
                        E::unpack(__builtin_nontemporal_load(src + j * 64), v[j]);
                    } else {
#pragma unroll
                        for (int e = 0; e < VEC; ++e) v[j][e] = id;
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < U; ++j)
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const uint32_t i = scan_layout::elem_in_tile(j, lane, e, VEC);
                    v[j][e] = i < rem ? E::load1(tin + i) : id;
                }
        }
#pragma unroll
        for (int j = 0; j < U; ++j) scan_vec(v[j], run);
        // Materialise the scanned values here: left alone, the compiler sinks the last addition of
        // every element past the look-back loop and keeps two extra values per chunk live across it.
#pragma unroll
        for (int j = 0; j < U; ++j)
#pragma unroll
            for (int e = 0; e < VEC; ++e) asm volatile("" : "+v"(v[j][e]));
    }
    // Group combine: each wave's prefix within the group and the group total; wave 0 publishes
    // and runs the look-back (publish and look_back take the lane from threadIdx.x: wave 0 only).
    // The barriers order the exchange line's writes before its reads within the workgroup.
    if (lane == 0) s_tot[wave] = run;
    __syncthreads();
    Acc wpre = id, gtot = id;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const Acc t = s_tot[w];
        if (w < (int)wave) wpre = op(wpre, t);
        gtot = op(gtot, t);
    }
    if (wave == 0) {
        Acc gex = id;
        if (group == 0) {
            publish(st.pre, group, gtot, st.tag_pre);
            if (lane == 0) *st.epoch_word = st.epoch;   // scan status: the workspace's latest call
        } else {
            publish(st.agg, group, gtot, st.tag_agg);
            gex = look_back<Acc>(st, group, op);
            publish(st.pre, group, op(gex, gtot), st.tag_pre);
        }
        if (lane == 0) *s_excl = gex;
    }
    __syncthreads();
    const Acc excl = op(*s_excl, wpre);
    if (!live) return;
    Out* tout = out + base;
    if constexpr (kVec) {
        constexpr int kWords = (int)(sizeof(Out) * VEC / 16);
        u32x4* dst = (u32x4*)tout + lane * kWords;
        Acc run2 = id;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            Acc x[VEC];
            if constexpr (kRaw) {   // the tile's scan, vector by vector from the loaded tile
                E::unpack(r[j], x);
                scan_vec(x, run2);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) x[e] = v[j][e];
            }
            if (scan_layout::vec_live(full, j, lane, rem, VEC)) {
                Out o[VEC];
#pragma unroll
                for (int e = 0; e < VEC; ++e) o[e] = (Out)op(excl, x[e]);
#pragma unroll
                for (int w = 0; w < kWords; ++w) {
                    u32x4 q;
                    __builtin_memcpy(&q, (const char*)o + 16 * w, 16);
                    __builtin_nontemporal_store(q, dst + j * 64 * kWords + w);
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < U; ++j)
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint32_t i = scan_layout::elem_in_tile(j, lane, e, VEC);
                if (i < rem) tout[i] = (Out)op(excl, v[j][e]);
            }
    }
}

// The last n % VEC (< VEC) elements of an aligned call, after scan_tiles has published every
// group's inclusive prefix: lane 0 continues the running value from the last group's prefix.
template <int DT, class Op>
__global__ __launch_bounds__(64) void scan_tail(const void* __restrict__ in_, size_t from, size_t n,
                                                 void* __restrict__ out_, ScanState st, size_t ngroups) {
    using E = Elem<DT>;
    using Acc = typename E::Acc;
    using Out = typename E::Out;
    const typename E::In* in = (const typename E::In*)in_;
    Out* out = (Out*)out_;
    Op op;
    Acc acc = Op::template identity<Acc>();
    bool ok = true;
    if (ngroups > 0) ok = read_slot<Acc>(st.pre, (long long)ngroups - 1, st.tag_pre, acc);
    if (threadIdx.x == 0) {
        if (ngroups == 0) *st.epoch_word = st.epoch;   // no scan_tiles launch: this call's epoch here
        if (!ok) __hip_atomic_store(st.error, st.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (size_t i = from; i < n; ++i) {
            acc = op(acc, E::load1(in + i));
            out[i] = (Out)acc;
        }
    }
}

template <int DT, bool kVec>
size_t scan_tiles_for(size_t n) {
    return scan_layout::tiles_for(n, ScanElem<DT>::VEC, scan_u<DT, kVec>());
}

// Tile count the workspace is sized for: the misaligned (smaller) tiles', the larger count.
size_t scan_ntiles(size_t n, int dtype) {
    switch (dtype) {
        case CDNA4_F32: return scan_tiles_for<CDNA4_F32, false>(n);
        case CDNA4_I32: return scan_tiles_for<CDNA4_I32, false>(n);
        case CDNA4_F64: return scan_tiles_for<CDNA4_F64, false>(n);
        case CDNA4_I64: return scan_tiles_for<CDNA4_I64, false>(n);
        case CDNA4_F16: return scan_tiles_for<CDNA4_F16, false>(n);
        case CDNA4_BF16: return scan_tiles_for<CDNA4_BF16, false>(n);
        default: return 0;
    }
}

// Workspace layout (scan_layout.hpp): [error: u32, padded to 256 B][agg: ntiles x 2 words]
// [pre: ntiles x 2 words] (64-bit values use both words of a tile, 32-bit values the first).
size_t scan_ws_bytes(size_t ntiles) { return scan_layout::ws_bytes(ntiles); }

template <int DT, class Op>
int scan_launch(const void* in, size_t n, void* out, void* ws, hipStream_t s) {
    using Acc = typename Elem<DT>::Acc;
    constexpr size_t VEC = ScanElem<DT>::VEC;
    if (n == 0) return 0;
    if (scan_tiles_for<DT, false>(n) > 0x7fffffffull) return CDNA4_ERR_INVALID_VALUE;
    // 16-byte aligned calls scan the whole vectors in scan_tiles and the last n % VEC elements
    // in scan_tail; misaligned calls scan everything element by element in scan_tiles.
    const bool vec = ((uintptr_t)in % 16) == 0 && ((uintptr_t)out % 16) == 0;
    const size_t n_main = scan_layout::main_elems(n, vec, (int)VEC);
    const size_t ntiles = vec ? scan_tiles_for<DT, true>(n_main) : scan_tiles_for<DT, false>(n_main);
    constexpr int kWaves = scan_group_waves<DT>();
    const size_t ngroups = scan_layout::groups_for(ntiles, kWaves);   // look-back slots: one per group
    char* w = (char*)ws;
    ScanState st;
    st.error = (uint32_t*)w;
    st.epoch_word = (uint32_t*)w + 1;
    st.epoch = scan_epoch();
    st.tag_agg = ((uint64_t)st.epoch << 2) | 1u;
    st.tag_pre = ((uint64_t)st.epoch << 2) | 2u;
    st.spin_limit = scan_spin_limit();
    st.agg = (uint64_t*)(w + scan_layout::agg_offset());
    st.pre = (uint64_t*)(w + scan_layout::pre_offset(ngroups));
    st.xchg = (unsigned char*)w + scan_layout::xchg_offset(ngroups);
    constexpr unsigned kThreads = 64 * kWaves;
    if (ngroups > 0) {
        if (vec)
            scan_tiles<DT, Op, true><<<(unsigned)ngroups, kThreads, 0, s>>>(in, n_main, out, st);
        else
            scan_tiles<DT, Op, false><<<(unsigned)ngroups, kThreads, 0, s>>>(in, n_main, out, st);
    }
    if (n_main < n) scan_tail<DT, Op><<<1, 64, 0, s>>>(in, n_main, n, out, st, ngroups);
    return launch_status();
}

template <template <int, class> class F, int DT>
int by_op(int op, const void* in, size_t n, void* out, void* ws, hipStream_t s) {
    switch (op) {
        case CDNA4_OP_SUM: return F<DT, OpSum>::run(in, n, out, ws, s);
        case CDNA4_OP_MAX: return F<DT, OpMax>::run(in, n, out, ws, s);
        case CDNA4_OP_MIN: return F<DT, OpMin>::run(in, n, out, ws, s);
        default: return CDNA4_ERR_INVALID_VALUE;
    }
}
template <template <int, class> class F>
int by_dtype(int op, int dtype, const void* in, size_t n, void* out, void* ws, hipStream_t s) {
    switch (dtype) {
        case CDNA4_F32: return by_op<F, CDNA4_F32>(op, in, n, out, ws, s);
        case CDNA4_I32: return by_op<F, CDNA4_I32>(op, in, n, out, ws, s);
        case CDNA4_F64: return by_op<F, CDNA4_F64>(op, in, n, out, ws, s);
        case CDNA4_I64: return by_op<F, CDNA4_I64>(op, in, n, out, ws, s);
        case CDNA4_F16: return by_op<F, CDNA4_F16>(op, in, n, out, ws, s);
        case CDNA4_BF16: return by_op<F, CDNA4_BF16>(op, in, n, out, ws, s);
        default: return CDNA4_ERR_INVALID_VALUE;
    }
}
template <int DT, class Op> struct ReduceF { static int run(const void* i, size_t n, void* o, void* w, hipStream_t s) { return reduce_launch<DT, Op>(i, n, o, w, s); } };
template <int DT, class Op> struct ScanF { static int run(const void* i, size_t n, void* o, void* w, hipStream_t s) { return scan_launch<DT, Op>(i, n, o, w, s); } };

bool valid_dtype(int dtype) { return dtype >= CDNA4_F32 && dtype <= CDNA4_I64; }
bool valid_op(int op) { return op >= CDNA4_OP_SUM && op <= CDNA4_OP_MIN; }

}  // namespace
}  // namespace cdna4

using namespace cdna4;

extern "C" size_t cdna3_reduce_workspace_size(size_t /*n*/, int /*dtype*/) {
    return ((size_t)kReduceMaxBlocks * (kReduceThreads / 64) + kReduce2Threads / 64) * 8;
}

extern "C" int cdna3_reduce(int op, int dtype, const void* in, size_t n, void* out, void* workspace,
                            size_t ws_bytes, cdna4_stream_t stream) {
    if (!valid_op(op) || !valid_dtype(dtype) || out == nullptr || (n > 0 && in == nullptr)) return CDNA4_ERR_INVALID_VALUE;
    if (workspace == nullptr || ws_bytes < cdna3_reduce_workspace_size(n, dtype)) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    return by_dtype<ReduceF>(op, dtype, in, n, out, workspace, (hipStream_t)stream);
}

extern "C" size_t cdna3_scan_workspace_size(size_t n, int dtype) {
    return scan_ws_bytes(scan_ntiles(n, dtype));
}

extern "C" int cdna3_scan_inclusive(int op, int dtype, const void* in, size_t n, void* out, void* workspace,
                                    size_t ws_bytes, cdna4_stream_t stream) {
    if (!valid_op(op) || !valid_dtype(dtype)) return CDNA4_ERR_INVALID_VALUE;
    if (n == 0) return 0;
    if (in == nullptr || out == nullptr || workspace == nullptr || ws_bytes < cdna3_scan_workspace_size(n, dtype))
        return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    return by_dtype<ScanF>(op, dtype, in, n, out, workspace, (hipStream_t)stream);
}

extern "C" int cdna3_scan_status(const void* workspace, int* status, cdna4_stream_t stream) {
    if (workspace == nullptr || status == nullptr) return CDNA4_ERR_INVALID_VALUE;
    if (int e = check_device()) return e;
    // words 0 and 1 of the workspace: the epoch of a call whose look-back gave up, the epoch of the
    // latest call; equal (and set) only when the latest call gave up
    uint32_t words[2] = {0u, 0u};
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(words, workspace, sizeof(words), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return (int)e;
    *status = (words[1] != 0u && words[0] == words[1]) ? 1 : 0;
    return 0;
}
