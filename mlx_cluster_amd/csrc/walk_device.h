// Device-side building blocks of the random-walk kernels (gfx950): the
// Philox4x32-10 generator, the reference's float32 index rule, CSR row reads
// with bounds checks, the per-wavefront walk queue, the per-lane windows for
// the rand stream (in LDS) and the output stream (in registers, stored by the
// wavefront together), and the edge-record layout.
//
// Reference semantics (vinayhpandya/mlx_cluster):
//   uniform walk   /root/reference/random_walks/RandomWalk.cpp:41-60
//   node2vec walk  /root/reference/random_walks/BiasedRandomWalk.cpp:20-28,52-100
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "mlxc.h"

namespace mlxc {

constexpr int kBlock = 256;           // 4 wavefronts of 64
constexpr int kWave = 64;
// Walks a wavefront takes from the global counter per atomic.  Ids taken
// but not started wait for a lane of that wavefront to free up, so at the
// end of a call a wavefront holding k per lane runs up to k walks in a row
// while others idle: 64, one per lane, cut that tail against 256 (same box:
// C3 10.73 -> 10.01 ms, C2 7.35 -> 7.24, C4 6.25 -> 6.16, C5x 16.86 -> 16.63).
// queue_take needs at least one id per lane from a single chunk.
constexpr int64_t kQueueChunk = 64;

// ------------------------------------------------------------------ Philox

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with a Weyl
// key schedule.  Each product is one v_mad_u64_u32 (both halves at once; a
// 32-bit multiply is quarter rate, and separate low and high multiplies cost
// two), and each three-way XOR one v_bitop3_b32 (gfx950; truth table 0x96).
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ void philox4x32_10(uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                              uint32_t& c3, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t n0 = xor3(static_cast<uint32_t>(p1 >> 32), c1, k0);
        const uint32_t n2 = xor3(static_cast<uint32_t>(p0 >> 32), c3, k1);
        c0 = n0;
        c1 = static_cast<uint32_t>(p1);
        c2 = n2;
        c3 = static_cast<uint32_t>(p0);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// 24 random bits -> float in [0, 1 - 2^-24]; both steps are exact.
__device__ __forceinline__ float unit_float(uint32_t x) {
    return static_cast<float>(x >> 8) * 0x1p-24f;
}

// --------------------------------------------------------- index selection

// RandomWalk.cpp:51-53: idx = (int64_t)(r * (row_end - row_start)) with r a
// float, i.e. the degree is rounded to float32, multiplied in float32 (RN)
// and truncated.  Clamped to [0, deg-1]: for r in [0,1) and deg <= 2^24 the
// clamp never fires; it keeps out-of-range r (and deg > 2^24, where
// (float)deg can round up) inside the row instead of reading past it.
__device__ __forceinline__ int64_t pick_index(float r, int64_t deg) {
    if (deg <= (int64_t{1} << 24)) {
        const float fdeg = static_cast<float>(static_cast<int32_t>(deg));  // exact
        const float p = __fmul_rn(r, fdeg);
        if (!(p >= 0.0f)) return 0;        // negative or NaN
        if (p >= fdeg) return deg - 1;     // r >= 1
        return static_cast<int64_t>(static_cast<int32_t>(p));
    }
    const float fdeg = static_cast<float>(deg);
    const float p = __fmul_rn(r, fdeg);
    if (!(p >= 0.0f)) return 0;
    if (p >= 9.0e18f) return deg - 1;
    const int64_t idx = static_cast<int64_t>(p);
    return idx < deg ? idx : deg - 1;
}

// rowptr[v], rowptr[v+1] as one 16-byte load (8-byte aligned).
struct RowBounds {
    int64_t begin, end;
};

__device__ __forceinline__ RowBounds load_row(const int64_t* __restrict__ rowptr, int64_t v) {
    typedef int64_t i64x2 __attribute__((ext_vector_type(2), aligned(8)));
    const i64x2 b = *reinterpret_cast<const i64x2*>(rowptr + v);
    return {b.x, b.y};
}

__device__ __forceinline__ bool node_ok(int64_t v, int64_t num_nodes) {
    return static_cast<uint64_t>(v) < static_cast<uint64_t>(num_nodes);
}

__device__ __forceinline__ bool row_ok(RowBounds r, int64_t num_edges) {
    return r.begin >= 0 && r.end >= r.begin && r.end <= num_edges;
}

// ------------------------------------------------------------ walk queue

// Per-wavefront queue of walk ids.  Lanes that need a walk vote; the wave
// hands out consecutive ids from its current chunk and takes a new chunk of
// kQueueChunk ids from the global counter with one atomic when the chunk runs
// dry.  All values here are wave-uniform.
struct WaveQueue {
    int64_t next, end;
};

__device__ __forceinline__ int64_t wave_bcast(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int lane_rank(uint64_t mask) {
    // number of set bits of mask below this lane
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

static_assert(kQueueChunk >= kWave, "one chunk must serve every lane of a wavefront");

// Returns the walk id for lanes with need == true (others get -1).
__device__ __forceinline__ int64_t queue_take(WaveQueue& q, bool need,
                                              unsigned long long* counter) {
    const uint64_t mask = __ballot(need);
    if (mask == 0) return -1;
    const int cnt = __popcll(mask);
    const int rank = lane_rank(mask);
    const int64_t avail = q.end - q.next;
    int64_t id;
    if (cnt <= avail) {
        id = q.next + rank;
        q.next += cnt;
    } else {
        // The lowest active lane takes the chunk; readfirstlane returns that
        // same lane's value, whatever the exec mask.
        const uint64_t active = __ballot(true);
        int64_t base = 0;
        if (static_cast<int>(__lane_id()) == __ffsll(static_cast<long long>(active)) - 1)
            base = static_cast<int64_t>(atomicAdd(counter, static_cast<unsigned long long>(kQueueChunk)));
        base = wave_bcast(base);
        id = rank < avail ? q.next + rank : base + (rank - avail);
        q.next = base + (cnt - avail);
        q.end = base + kQueueChunk;
    }
    return need ? id : -1;
}

// Arguments shared by the walk kernels.
struct WalkArgs {
    const int64_t* rowptr;
    const int64_t* col;
    const int64_t* start;
    const float* rand;
    void* n_out;    // OutT [num_walks, walk_length + 1]
    void* e_out;    // OutT [num_walks, walk_length] or null
    int64_t* work;  // [0] status bits, [1] walk-queue counter
    int64_t num_nodes;
    int64_t num_edges;
    int64_t num_walks;
    int32_t walk_length;
    uint32_t key0, key1;  // Philox key (the seed) when the kernel generates its uniforms
    // Philox walk index of walk 0 of this call: walk n draws from the stream
    // of walk walk_base + n, so a call over any slice of a larger batch gives
    // that slice's walks.  Generated uniform streams only (0 with a rand tensor).
    int64_t walk_base;
};

// ------------------------------------------------- stream windows

// Per-lane windows for the two streams of the uniform walk (rand: LdsWindow
// below, in LDS; output: OutWin, in registers).
//
// The rand stream: walk n reads rand[n*L + l] at step l, so a lane walks
// through its own row 4 bytes at a time while its 63 neighbours do the same
// 4*L bytes apart.  Read one float at a time, nearly every step misses L2 and
// costs a 128-byte line.  Instead each slot keeps the next RW floats of its
// row at hand (in LDS, LdsWindow below), loaded as one aligned RW*4-byte
// block, so the stream costs one line per RW steps.
//
// The output: walk n writes n_out[n*(L+1) + j] for j = 0..L, one 8-byte entry
// per step.  Scattered 8-byte stores reach memory as partial 32-byte writes.
// Each slot buffers its entries in an 8-entry window aligned to 64 bytes of
// the output (OutWin below) and the wavefront stores completed windows, and
// the constant tails of walks that sink in a node of out-degree 0, as whole
// 64-byte blocks where they can (the partial blocks at the ends of rows and
// tails from consecutive lanes, one write each).  The whole blocks are
// non-temporal: the output is never read back, and streaming it past the
// caches keeps them for the graph.
// One block of RW uniforms as read or generated, before it is stored.
template <int RW>
struct RandWindow {
    float w[RW];
};

// First index of the rand block that serves rand[f]: the aligned block, or for
// the array's last partial block the last RW values (total must be a multiple
// of 4 and at least RW, so every block is 16-byte aligned and in bounds).
template <int RW>
__device__ __forceinline__ int64_t rw_block_base(int64_t f, int64_t total) {
    const int64_t base = f & ~static_cast<int64_t>(RW - 1);
    return base + RW <= total ? base : total - RW;
}

template <int RW>
__device__ __forceinline__ void rw_load_at(RandWindow<RW>& r, const float* __restrict__ rand,
                                           int64_t base) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4* p = reinterpret_cast<const f32x4*>(rand + base);
#pragma unroll
    for (int i = 0; i < RW / 4; ++i) {
        const f32x4 x = __builtin_nontemporal_load(p + i);
        r.w[4 * i] = x.x;
        r.w[4 * i + 1] = x.y;
        r.w[4 * i + 2] = x.z;
        r.w[4 * i + 3] = x.w;
    }
}

// Uniform i of the seeded stream, in the layout of mlxc_philox_uniform:
// word i % 4 of Philox(counter = (i / 4 lo, i / 4 hi, 0, 0), key).
__device__ __forceinline__ float philox_uniform_at(int64_t i, uint32_t k0, uint32_t k1) {
    const uint64_t j = static_cast<uint64_t>(i) >> 2;
    uint32_t c0 = static_cast<uint32_t>(j), c1 = static_cast<uint32_t>(j >> 32), c2 = 0, c3 = 0;
    philox4x32_10(c0, c1, c2, c3, k0, k1);
    const int w = static_cast<int>(i & 3);
    return unit_float(w == 0 ? c0 : w == 1 ? c1 : w == 2 ? c2 : c3);
}

// Generates the block of the seeded stream starting at base (a multiple of 4).
template <int RW>
__device__ __forceinline__ void rw_gen_at(RandWindow<RW>& r, int64_t base, uint32_t k0,
                                          uint32_t k1) {
#pragma unroll
    for (int i = 0; i < RW / 4; ++i) {
        const uint64_t j = (static_cast<uint64_t>(base) >> 2) + i;
        uint32_t c0 = static_cast<uint32_t>(j), c1 = static_cast<uint32_t>(j >> 32), c2 = 0, c3 = 0;
        philox4x32_10(c0, c1, c2, c3, k0, k1);
        r.w[4 * i] = unit_float(c0);
        r.w[4 * i + 1] = unit_float(c1);
        r.w[4 * i + 2] = unit_float(c2);
        r.w[4 * i + 3] = unit_float(c3);
    }
}

// Block start for rand[f].  A generated stream has no array end to respect;
// its uniform f is stream position f + off (off = walk_base * walk_length),
// and its blocks are aligned in stream positions, so the block start may lie
// before f = 0 (a negative index, never read: the block is generated).
template <int RW, bool kGen>
__device__ __forceinline__ int64_t rw_base(int64_t f, int64_t total, int64_t off) {
    return kGen ? ((f + off) & ~static_cast<int64_t>(RW - 1)) - off : rw_block_base<RW>(f, total);
}

// Fills the window with the block that serves rand[f], read or generated.
template <int RW, bool kGen>
__device__ __forceinline__ void rw_fetch(RandWindow<RW>& r, const WalkArgs& a, int64_t f,
                                         int64_t total, int64_t off) {
    if (kGen) rw_gen_at(r, rw_base<RW, kGen>(f, total, off) + off, a.key0, a.key1);
    else rw_load_at(r, a.rand, rw_base<RW, kGen>(f, total, off));
}

// The walk loops keep each slot's rand window in LDS rather than in
// registers: a register window must be shifted on every pick and is copied on
// every control path that changes it, which made the loops VALU-bound.  The
// area is uniform-major ([position][thread]), so the lanes of a wavefront
// reading the same position, or any positions, hit distinct banks.  A block
// arrives in registers (rw_fetch) and is stored once; each pick reads one
// float.
template <int RW>
struct LdsWindow {
    int32_t pos;    // position of the next uniform
    int32_t valid;  // uniforms left from pos
};

// Stores a fetched block whose first k entries precede the walk's next uniform.
template <int RW>
__device__ __forceinline__ void lw_store(float (&area)[RW][kBlock], LdsWindow<RW>& lw,
                                         const RandWindow<RW>& blk, int k) {
#pragma unroll
    for (int i = 0; i < RW; ++i) area[i][threadIdx.x] = blk.w[i];
    lw.pos = k;
    lw.valid = RW - k;
}

// The next uniform of the window (valid > 0).
template <int RW>
__device__ __forceinline__ float lw_take(float (&area)[RW][kBlock], LdsWindow<RW>& lw) {
    static_assert((RW & (RW - 1)) == 0, "RW is a power of two");
    const float r = area[lw.pos & (RW - 1)][threadIdx.x];
    lw.pos += 1;
    lw.valid -= 1;
    return r;
}

// Output rows are written in blocks of 8 entries, aligned in the output: 64
// bytes of int64 entries, or 32 bytes with the compact int32 output.  A lane
// buffers its walk's entries in an OutWin.  The stores of a completed block,
// and of the run of entries that a walk absorbed by a sink repeats to the end
// of its row, are deferred to ow_drain, which the whole wavefront executes
// together: completed blocks are staged through LDS and stored by several
// lanes per block, one 16-byte non-temporal store each, and the whole blocks
// of a run are stored by the whole wavefront in consecutive 16-byte pieces.
// Every such store instruction covers whole blocks and the L2 sends one full
// write per block; a lane storing its own 64-byte block in four pieces leaves
// up to four partial writes of it (measured: 3.6 write requests per block on
// MI355X, against 1.0 here).  The partial blocks at the two ends of a row, and
// a run's entries before its first block boundary and after its last whole
// block, are stored the same way, one entry per lane on consecutive lanes, so
// that each is one write request instead of one per entry: eight partial
// blocks per store instruction, and a run's two ends in one; and a walk
// absorbed by a sink fills its row from its current entry as one run.
// Against the same partial entries stored by their own lanes one at a time
// (up to eight store instructions, a write request each), the fill's first
// entries pushed through the window, on MI355X: configuration 4 6.15 -> 5.76
// ms (62% of its walks meet a sink, and its rows of 21 entries have partial
// blocks at both ends), 2 7.24 -> 7.14, 2 with the int32 output 6.74 -> 6.62,
// 3 10.00 -> 9.88, 5x 16.57 -> 16.47.
//
// Every output store is issued by ow_drain, which the walk loops call right
// after issuing their reads and before their single wait.  No store is then
// in flight when a loop iteration begins and reuses registers: on gfx9 vmcnt
// counts stores too, and the compiler makes a register that a pending store
// reads wait for that store.
//
// Between a completion and the drain the window is not pushed again: each
// iteration of the walk loops pushes at most one entry per window, and a fill
// in the same iteration flushes only what that push left (a push that
// completes a block leaves nothing), so a window defers at most one block
// and one run per drain.
//
// T is the type the entries are buffered in (int32_t: the windowed walks'
// node and edge ids fit in it); OutT is the output element type, int64_t (the
// reference's layout) or int32_t.

// Cache policy of the two kinds of output store.  Whole blocks stream past
// the caches (non-temporal).  The partial blocks at the ends of a row are
// shared with the neighbouring row, which another lane writes at about the
// same time (walks are taken in order), so they are stored through L2, where
// the two parts merge into one write.  Measured on MI355X against
// non-temporal partial stores: 3% faster at configuration 2, 7% at 4 (rows of
// 21 entries) and 18% at 5 (31 entries).
#ifndef MLXC_BLOCK_NT
#define MLXC_BLOCK_NT 1
#endif
#ifndef MLXC_PARTIAL_NT
#define MLXC_PARTIAL_NT 0
#endif

// 16 bytes of output entries: 2 int64 or 4 int32.
template <typename OutT>
struct Vec16;
template <>
struct Vec16<int64_t> {
    typedef int64_t type __attribute__((ext_vector_type(2)));
    static constexpr int kLanes = 2;
};
template <>
struct Vec16<int32_t> {
    typedef int32_t type __attribute__((ext_vector_type(4)));
    static constexpr int kLanes = 4;
};

// The output stores go through global-address-space pointers.  The drain's
// destinations come back from LDS staging or from another lane's registers,
// where the compiler cannot tell them from LDS addresses, and would emit flat
// stores, which also count in lgkmcnt: every later wait for an LDS read or a
// scalar load would then wait for the stores as well.  (No time difference
// measured on MI355X: the loop's single wait covers the stores either way.)
template <typename T>
using GlobalPtr = __attribute__((address_space(1))) T*;

template <typename OutT>
__device__ __forceinline__ void store_block_part(typename Vec16<OutT>::type v, OutT* p) {
    typedef typename Vec16<OutT>::type V;
    GlobalPtr<V> q = (GlobalPtr<V>)(p);
    if (MLXC_BLOCK_NT) __builtin_nontemporal_store(v, q);
    else *q = v;
}

template <typename OutT>
__device__ __forceinline__ void store_partial(OutT v, OutT* p) {
    GlobalPtr<OutT> q = (GlobalPtr<OutT>)(p);
    if (MLXC_PARTIAL_NT) __builtin_nontemporal_store(v, q); else *q = v;
}

// Entries p[0 .. kLanes-1] (int32) widened to one 16-byte vector of OutT.
template <typename OutT>
__device__ __forceinline__ typename Vec16<OutT>::type vec16_from(const int32_t* p);
template <>
__device__ __forceinline__ Vec16<int64_t>::type vec16_from<int64_t>(const int32_t* p) {
    typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
    const i32x2 v = *reinterpret_cast<const i32x2*>(p);
    return Vec16<int64_t>::type{static_cast<int64_t>(v.x), static_cast<int64_t>(v.y)};
}
template <>
__device__ __forceinline__ Vec16<int32_t>::type vec16_from<int32_t>(const int32_t* p) {
    return *reinterpret_cast<const Vec16<int32_t>::type*>(p);
}

template <typename OutT>
__device__ __forceinline__ typename Vec16<OutT>::type vec16_splat(OutT x) {
    typename Vec16<OutT>::type v;
#pragma unroll
    for (int i = 0; i < Vec16<OutT>::kLanes; ++i) v[i] = x;
    return v;
}

template <typename T>
struct OutWin {
    T w[8];              // w[8-count .. 7] hold the newest entries; w[7] is entry g
    int count;
    // Deferred stores, written by ow_drain:
    void* blk;           // set: w[i] belongs at blk + i; the last blk_n entries are
    int32_t blk_n;       //   stored (8: a complete aligned block, by the wavefront)
    void* run;           // set: run_n entries of run_val from run, of which the
    int32_t run_n;       //   first run_head lie before the first block boundary
    int32_t run_head;
    T run_val;
};

template <typename T>
__device__ __forceinline__ void ow_init(OutWin<T>& o) {
    o.count = 0;
    o.blk = nullptr;
    o.blk_n = 0;
    o.run = nullptr;
    o.run_n = 0;
    o.run_head = 0;
    o.run_val = 0;
}

// Per-wavefront LDS staging of ow_drain.
struct WaveStage {
    int32_t vals[kWave][8];  // completed and partial blocks (entries as int32)
    void* dst[kWave];
    int32_t first[kWave];    // a partial block's first entry written
};

// Writes (defers to ow_drain) the buffered entries, the newest of which is
// output index g: a complete aligned block, or the partial block at an end
// of the row.
template <typename T, typename OutT>
__device__ __forceinline__ void ow_flush(OutWin<T>& o, OutT* __restrict__ out, int64_t g) {
    if (o.count > 0) {
        o.blk = out + (g - 7);  // only blk + 8 - blk_n .. blk + 7 is written
        o.blk_n = o.count;
    }
    o.count = 0;
}

// Appends the entry for output index g; completes the window's block when g
// closes a block.
template <typename T, typename OutT>
__device__ __forceinline__ void ow_push(OutWin<T>& o, OutT* __restrict__ out, int64_t g, T x) {
#pragma unroll
    for (int i = 0; i < 7; ++i) o.w[i] = o.w[i + 1];
    o.w[7] = x;
    o.count = o.count < 8 ? o.count + 1 : 8;
    if (((g + 1) & 7) == 0) ow_flush(o, out, g);
}

// Output indices g .. g_last (inclusive) all hold x; the window holds the
// entries before g, which are flushed.  The fill is left to ow_drain as a
// run: its entries before the first block boundary, its whole blocks and the
// entries after the last one.
template <typename T, typename OutT>
__device__ __forceinline__ void ow_fill(OutWin<T>& o, OutT* __restrict__ out, int64_t g,
                                        int64_t g_last, T x) {
    if (o.count) ow_flush(o, out, g - 1);
    if (g <= g_last) {
        const int64_t n = g_last + 1 - g;
        const int64_t head = (8 - (g & 7)) & 7;
        o.run = out + g;
        o.run_n = static_cast<int32_t>(n);
        o.run_head = static_cast<int32_t>(head < n ? head : n);
        o.run_val = x;
    }
}

// s_waitcnt vmcnt(0): every vector-memory operation of the wavefront has
// completed.  The walk loops wait once per iteration, unconditionally, after
// issuing their reads and while nothing else is pending; on every path around
// the loop no load is then left in flight, and the compiler needs no further
// wait where a register of an earlier load is reused.  (gfx9 encoding:
// vmcnt 0, expcnt 7, lgkmcnt 15.)
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Keeps a value in a VGPR up to this point: the pad word of a 16-byte record
// load is otherwise dead at once, and a register reused before the load
// returns forces a wait.
__device__ __forceinline__ void keep_vgpr(int32_t x) { asm volatile("" ::"v"(x)); }

// Compiler and LDS ordering point between the lanes of one wavefront (LDS
// operations of a wavefront execute in order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void* read_lane_ptr(void* p, int lane) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(u), lane);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(u >> 32), lane);
    return reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Stores the deferred blocks and runs of every lane's window into an output
// of OutT.  Must be reached by all lanes of the wavefront together
// (wave-uniform control flow); st is the wavefront's own staging area.
template <typename OutT, typename T>
__device__ __forceinline__ void ow_drain(OutWin<T>& o, WaveStage& st) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    static_assert(sizeof(T) == 4, "staged and broadcast as 32-bit entries");
    constexpr int kPer = Vec16<OutT>::kLanes;  // entries per 16-byte store
    constexpr int kParts = 8 / kPer;           // lanes per block: 4 (int64) or 2 (int32)
    const int lane = __lane_id();
    const int part = lane % kParts;
    const bool full = o.blk != nullptr && o.blk_n == 8;
    const bool partial = o.blk != nullptr && !full;  // a partial block at an end of a row
    const uint64_t blocks = __ballot(full);
    const uint64_t partials = __ballot(partial);
    if (blocks | partials) {
        // staged in rank order: the complete blocks, then the partial ones
        if (o.blk != nullptr) {
            const int rank = full ? lane_rank(blocks) : __popcll(blocks) + lane_rank(partials);
            *reinterpret_cast<i32x4*>(&st.vals[rank][0]) =
                i32x4{static_cast<int32_t>(o.w[0]), static_cast<int32_t>(o.w[1]),
                      static_cast<int32_t>(o.w[2]), static_cast<int32_t>(o.w[3])};
            *reinterpret_cast<i32x4*>(&st.vals[rank][4]) =
                i32x4{static_cast<int32_t>(o.w[4]), static_cast<int32_t>(o.w[5]),
                      static_cast<int32_t>(o.w[6]), static_cast<int32_t>(o.w[7])};
            st.dst[rank] = o.blk;
            st.first[rank] = 8 - o.blk_n;
        }
        wave_sync();
        const int c = __popcll(blocks);
        for (int r = 0; r < c; r += kWave / kParts) {  // kWave / kParts blocks per store
            const int k = r + lane / kParts;
            if (k < c)
                store_block_part(vec16_from<OutT>(&st.vals[k][kPer * part]),
                                 static_cast<OutT*>(st.dst[k]) + kPer * part);
        }
        // partial blocks: eight lanes per block, lane i storing entry i when
        // it is one of the block's, eight blocks per store instruction
        const int cp = __popcll(partials);
        for (int r = 0; r < cp; r += kWave / 8) {
            const int k = c + r + lane / 8;
            const int i = lane % 8;
            if (r + lane / 8 < cp && i >= st.first[k])
                store_partial(static_cast<OutT>(st.vals[k][i]), static_cast<OutT*>(st.dst[k]) + i);
        }
        wave_sync();
    }
    o.blk = nullptr;
    uint64_t runs = __ballot(o.run_n > 0);
    while (runs) {  // wave-uniform: one lane's run at a time, the whole wave storing it
        const int src = __builtin_ctzll(runs);
        runs &= runs - 1;
        OutT* dst = static_cast<OutT*>(read_lane_ptr(o.run, src));
        const int32_t n = __builtin_amdgcn_readlane(o.run_n, src);
        const int32_t head = __builtin_amdgcn_readlane(o.run_head, src);
        const int32_t blocks_n = (n - head) >> 3;
        const int32_t tail = n - head - 8 * blocks_n;
        const OutT x = static_cast<OutT>(
            static_cast<T>(__builtin_amdgcn_readlane(static_cast<int32_t>(o.run_val), src)));
        const typename Vec16<OutT>::type xx = vec16_splat(x);
        OutT* body = dst + head;  // a block boundary
        for (int c = lane; c < kParts * blocks_n; c += kWave) store_block_part(xx, body + kPer * c);
        // the entries before the first block boundary and after the last
        // whole block, one per lane
        if (lane < head + tail)
            store_partial(x, lane < head ? dst + lane : body + 8 * static_cast<int64_t>(blocks_n) + (lane - head));
    }
    o.run = nullptr;
    o.run_n = 0;
}

// ----------------------------------------------------------- edge records

// One record per CSR entry e, written by edge_record_kernel at the start of
// each call: the target node col[e] together with its row bounds.  A walk at
// node v with row [begin, begin + deg) picks e and reads record e: one
// dependent 16-byte read per step gives the next node and everything needed
// for the step after it, where the plain CSR needs two (rowptr[v], then
// col[e]).  The walk's random reads, which bound it, halve; the records cost
// 16 bytes per edge of HBM and one pass over the graph per call.
struct __attribute__((aligned(16))) EdgeRecord {
    int32_t node;   // col[e]
    int32_t begin;  // rowptr[col[e]]
    int32_t deg;    // rowptr[col[e] + 1] - rowptr[col[e]]; < 0 marks a malformed entry
    int32_t pad;
};

constexpr int32_t kRecBadNode = -1;  // col[e] outside [0, num_nodes)
constexpr int32_t kRecBadRow = -2;   // row of col[e] outside [0, num_edges] or decreasing
constexpr int32_t kRecLongRow = -3;  // packed records: a row too long for the degree field

// The uniform walk's edge record packed into 8 bytes, for graphs whose ids
// leave at least kPackedMinDegreeBits for the degree.  With c the bits of
// num_nodes - 1, s those of num_edges and d = min(24, 64 - c - s): bits
// [0, d) hold a degree code, [d, d + s) the row begin and [64 - c, 64) the
// node.  The code is the degree + 3; codes 2 and 1 mark a bad node and a bad
// row, and code 0 a row longer than the field holds, whose end the walk then
// reads from rowptr.  A 128-byte line holds 16 records instead of 8, so twice
// the share of the graph stays in each XCD's L2 and in the Infinity Cache.
// A degree the code holds is below 2^24, where the float32 index rule is
// exact (pick_index).
constexpr int kPackedMinDegreeBits = 16;
struct PackedFormat {
    static constexpr int kMaxDegreeBits = 24;
    static constexpr int32_t kMaxInlineDegree = (1 << kMaxDegreeBits) - 4;
    int32_t c;  // node bits, 1 .. 31
    int32_t s;  // row-begin bits, 1 .. 31
    int32_t d;  // degree-code bits, kPackedMinDegreeBits .. kMaxDegreeBits

    __host__ __device__ uint64_t pack(int32_t node, int32_t begin, int32_t deg) const {
        const uint32_t most = (1u << d) - 4;  // the largest degree the code holds
        const uint32_t code = deg < 0 ? static_cast<uint32_t>(deg + 3)  // kRecBadNode, kRecBadRow
                              : static_cast<uint32_t>(deg) > most ? 0u   // kRecLongRow
                                                                  : static_cast<uint32_t>(deg) + 3;
        return (static_cast<uint64_t>(static_cast<uint32_t>(node) & ((1u << c) - 1)) << (64 - c)) |
               (static_cast<uint64_t>(static_cast<uint32_t>(begin)) << d) | code;
    }

    // deg: the degree, or kRecBadNode / kRecBadRow / kRecLongRow.  Five VALU
    // operations: a shift, two masks, a funnel shift (v_alignbit_b32) and
    // the subtraction.
    __device__ __forceinline__ void unpack(uint64_t x, int32_t& node, int32_t& begin,
                                           int32_t& deg) const {
        const uint32_t lo = static_cast<uint32_t>(x), hi = static_cast<uint32_t>(x >> 32);
        node = static_cast<int32_t>(hi >> (32 - c));
        begin = static_cast<int32_t>(__builtin_amdgcn_alignbit(hi, lo, d) & ((1u << s) - 1));
        deg = static_cast<int32_t>(lo & ((1u << d) - 1)) - 3;
    }
};

// Whether a graph's records pack into 8 bytes, and the field widths.
inline __host__ bool packed_format(int64_t num_nodes, int64_t num_edges, PackedFormat& f) {
    auto bits = [](int64_t x) {
        int b = 0;
        while (x > 0) { ++b; x >>= 1; }
        return b;
    };
    f.c = num_nodes > 2 ? bits(num_nodes - 1) : 1;
    f.s = num_edges > 1 ? bits(num_edges) : 1;
    f.d = 64 - f.c - f.s < PackedFormat::kMaxDegreeBits ? 64 - f.c - f.s
                                                         : PackedFormat::kMaxDegreeBits;
    return f.c <= 31 && f.s <= 31 && f.d >= kPackedMinDegreeBits;
}
// Search index of the node2vec walk over sorted rows: level 0 is col as
// int32 (col32); level k >= 1 holds col32[16^k * i] for every i.  Every
// level is padded to whole blocks of 16 entries (64 bytes).  Built by
// edge_record_kernel, read by node2vec_rec_kernel.
constexpr int kSearchBlock = 16;
constexpr int kMaxLevels = 8;  // 16^8 = 2^32 > any num_edges the records allow
struct IndexLevels {
    int32_t* level[kMaxLevels];
    int32_t count;  // levels in use; 0: no col32 (the uniform walk)
};

// Levels a graph of num_edges entries needs: the coarsest level k at which a
// row may have to start its search is msb(num_edges - 1) / 4.
inline __host__ __device__ int index_levels(int64_t num_edges) {
    if (num_edges <= 1) return 1;
    int msb = 0;
    for (int64_t x = num_edges - 1; x > 1; x >>= 1) ++msb;
    return msb / 4 + 1;
}

// Dense adjacency bitmaps of the node2vec record walk's hub rows: bit c of
// bitmap s is set when node c is in row(node_of[s]).  A membership test on a
// hub row then costs one read instead of a descent through the index levels
// (about log16(deg) + 1 reads).  The rows that get one are those of degree at
// least a threshold, the smallest power of two >= kHubMinDegree for which the
// rows that reach it fit the reserved slots; it is chosen on the device per
// call (hub_count_kernel, hub_assign_kernel).  The edge and start records
// carry the slot of their node in their pad word (-1: none).
constexpr int64_t kHubMinDegree = 256;
constexpr int kHubMinLog = 8;        // log2(kHubMinDegree)
constexpr int kHubDegreeClasses = 24;  // rows counted by floor(log2(deg)) - 8, capped
// info words: [0] the degree threshold (INT64_MAX: no bitmaps), [1] slots
// assigned, [2 + k] rows with floor(log2(deg)) - kHubMinLog == k (the last
// class also holds every larger degree)
constexpr int kHubInfoWords = 2 + kHubDegreeClasses;
struct HubBitmaps {
    int32_t* slot_of;  // [num_nodes]; written only for rows at or above the threshold
    int32_t* node_of;  // [max]
    uint32_t* bits;    // [max][words]
    int64_t* info;     // [kHubInfoWords]
    int64_t words;     // 32-bit words per bitmap: ceil(num_nodes / 32), rounded up to 4
    int32_t max;       // slots reserved; 0: no bitmaps
};

// Row hash tables of the node2vec record walk: an exact membership table per
// row of kHashMinSpan.. entries below kHashMaxDegree, so that "is t in
// row(x)" costs one 64-byte read instead of a descent through the index
// levels (two or three reads for such rows).  Row x of begin b and degree d
// has B = d / 8 + 1 buckets of kSearchBlock int32 slots (fewer than half of
// them used; one bucket, which holds the whole row, when d <= 16), starting
// at bucket b / 8 + x: the buckets of consecutive rows follow each other
// without overlap (b / 8 + x + B <= (b + d) / 8 + x + 1), and all of them
// lie below num_edges / 8 + num_nodes + 1.  Node t sits in
// bucket hash_bucket(t, B), or when that bucket was full at insertion, in the
// first bucket after it (cyclically) that was not; an empty slot holds -1.
// So a lookup reads bucket hash_bucket(t, B): t found answers yes, an empty
// slot no, and a full bucket without t sends it to the next bucket.
// A row gets a table when its search would take more than one read (it
// spans more than one aligned 16-entry block of col32) and it has no hub
// bitmap (degree below the call's hub threshold).
constexpr int32_t kHashMaxDegree = 1024;

__host__ __device__ __forceinline__ bool row_hashed(int64_t begin, int64_t deg,
                                                    int64_t hub_threshold) {
    return deg > 1 && deg < kHashMaxDegree && deg < hub_threshold &&
           ((begin ^ (begin + deg - 1)) >> 4) != 0;
}

__host__ __device__ __forceinline__ int32_t hash_buckets(int32_t deg) {
    return deg <= kSearchBlock ? 1 : (deg >> 3) + 1;
}

__host__ __device__ __forceinline__ int64_t hash_region(int32_t begin, int32_t node) {
    return (static_cast<int64_t>(begin) >> 3) + node;
}

// Bucket of node t among B: the high word of (t * golden ratio mod 2^32) * B
// (Fibonacci hashing: consecutive ids spread over the buckets).
__host__ __device__ __forceinline__ int32_t hash_bucket(int32_t t, int32_t buckets) {
    const uint32_t h = static_cast<uint32_t>(t) * 0x9E3779B1u;
    return static_cast<int32_t>((static_cast<uint64_t>(h) * static_cast<uint32_t>(buckets)) >> 32);
}

// Start records a preparation pass writes besides its edge pass: walk n's
// start node in the record format, into init[n].
struct StartRecords {
    const int64_t* start;
    int64_t num_walks;
    EdgeRecord* init;
};

constexpr size_t kRecordOffset = 256;  // bytes of workspace before the records

// Walks on graphs small enough for LDS (uniform_walk_lds_kernel,
// node2vec_lds_kernel): rowptr and col as int32 in each block's LDS, for
// calls bound by launch latency.  A workspace of kRecordOffset bytes (less
// than any record or start-record layout) selects them.
constexpr int kLdsGraphEntries = 14336;              // rowptr + col entries (56 KB)
// Threads per block of the LDS walks.  Every block first copies the whole
// graph, so the copy is the block's serial part: 1024 threads split it four
// times finer than 256 (the reference tests' 2,000 walks of 5 steps on the
// Cora-like graph: 11.2 -> 6.7 us per launch).
constexpr int kLdsBlock = 1024;
// Fewest walking threads per block of the node2vec LDS walk: one wavefront
// per SIMD of the block's compute unit.
constexpr int kLdsMinWalkers = 256;

constexpr int64_t kLdsWalkSteps = int64_t{1} << 20;  // calls of 1 .. 2^20 steps
__host__ __device__ inline bool lds_walk_fits(int64_t num_nodes, int64_t num_edges,
                                              int64_t num_walks, int64_t walk_length) {
    return num_nodes + 1 + num_edges <= kLdsGraphEntries && walk_length >= 1 &&
           num_walks <= kLdsWalkSteps && num_walks * walk_length <= kLdsWalkSteps;
}

}  // namespace mlxc
