// Random-walk kernels for MI355X (gfx950) and the C ABI declared in
// include/mlxc.h.
//
// Reference semantics (vinayhpandya/mlx_cluster):
//   uniform walk   /root/reference/random_walks/RandomWalk.cpp:41-60
//   node2vec walk  /root/reference/random_walks/BiasedRandomWalk.cpp:20-28,52-100
//
// Design: the walk is a chain of dependent random gathers (rowptr[v] pair,
// then col[e]), so throughput comes from the number of chains in flight, not
// from arithmetic.  Every lane runs a small state machine over W independent
// walk slots; each loop iteration issues the rowptr loads of all live slots,
// then their col loads, so a lane keeps W chains in flight.  A lane whose
// walk ends (or sinks in a node of out-degree 0, which absorbs the walk) takes
// the next walk from a per-wavefront queue refilled by one global atomic per
// kQueueChunk walks, so lanes never idle while walks remain and the kernel's
// tail is about one walk long.  The grid is the resident capacity of the
// device (persistent waves).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <string>

#include "mlxc.h"

namespace {

constexpr int kBlock = 256;          // 4 wavefronts of 64
constexpr int kWave = 64;
constexpr int64_t kQueueChunk = 256; // walks taken per global atomic

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

#define MLXC_HIP_TRY(expr)                                                          \
    do {                                                                            \
        hipError_t err_ = (expr);                                                   \
        if (err_ != hipSuccess)                                                     \
            return fail(MLXC_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(err_)); \
    } while (0)

// ------------------------------------------------------------------ Philox

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with a Weyl
// key schedule.
__device__ __forceinline__ void philox4x32_10(uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                              uint32_t& c3, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint32_t lo0 = 0xD2511F53u * c0;
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo1 = 0xCD9E8D57u * c2;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2);
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
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
        if (__lane_id() == __ffsll(static_cast<long long>(active)) - 1)
            base = static_cast<int64_t>(atomicAdd(counter, static_cast<unsigned long long>(kQueueChunk)));
        base = wave_bcast(base);
        id = rank < avail ? q.next + rank : base + (rank - avail);
        q.next = base + (cnt - avail);
        q.end = base + kQueueChunk;
    }
    return need ? id : -1;
}

// --------------------------------------------------------------- kernels

struct WalkArgs {
    const int64_t* rowptr;
    const int64_t* col;
    const int64_t* start;
    const float* rand;
    int64_t* n_out;
    int64_t* e_out;
    int64_t* work;  // [0] status bits, [1] walk-queue counter
    int64_t num_nodes;
    int64_t num_edges;
    int64_t num_walks;
    int32_t walk_length;
};

__global__ void zero_words_kernel(int64_t* p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0;
}

// Uniform walk: W walk slots per lane, walks from the wave queue.
template <int W, bool kEdges>
__global__ __launch_bounds__(kBlock) void uniform_walk_kernel(WalkArgs a) {
    const int64_t L = a.walk_length;
    const int64_t N = a.num_walks;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int64_t n[W], v[W], l[W];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) { n[s] = -1; l[s] = L; v[s] = 0; }

    while (true) {
        // Acquire walks for empty slots; write their first column.
        bool unretired = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = (n[s] < N) && (l[s] >= L);  // slot idle (or never used)
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;  // id >= N ends the slot for good
                if (id < N) {
                    const int64_t s0 = a.start[id];
                    a.n_out[id * (L + 1)] = s0;
                    v[s] = s0;
                    l[s] = 0;
                    if (!node_ok(s0, a.num_nodes)) {
                        status |= MLXC_STATUS_BAD_NODE;
                        for (int64_t j = 1; j <= L; ++j) a.n_out[id * (L + 1) + j] = s0;
                        if (kEdges)
                            for (int64_t j = 0; j < L; ++j) a.e_out[id * L + j] = -1;
                        l[s] = L;
                    }
                }
            }
            unretired |= (n[s] < N);
        }
        // The whole wave leaves together, once every slot of every lane has
        // drawn an id past the end; until then idle lanes keep voting.
        if (!__any(unretired)) break;

        // Phase 1: rowptr pair and the step's uniform, for every live slot.
        RowBounds rb[W];
        float r[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            rb[s] = {0, 0};
            r[s] = 0.0f;
            if (live) {
                rb[s] = load_row(a.rowptr, v[s]);
                r[s] = __builtin_nontemporal_load(a.rand + n[s] * L + l[s]);
            }
        }
        // Phase 2: candidate edge and its target, for every moving slot.
        int64_t e[W], x[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            e[s] = -1;
            x[s] = v[s];
            if (live) {
                const int64_t deg = rb[s].end - rb[s].begin;
                if (!row_ok(rb[s], a.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                } else if (deg > 0) {
                    e[s] = rb[s].begin + pick_index(r[s], deg);
                    x[s] = a.col[e[s]];
                }
            }
        }
        // Phase 3: store, advance, and finish sunk / broken walks.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            if (!live) continue;
            int64_t* out = a.n_out + n[s] * (L + 1);
            const bool moved = e[s] >= 0;
            bool stop = !moved;  // deg == 0 (absorbing) or malformed row
            out[l[s] + 1] = x[s];
            if (kEdges) a.e_out[n[s] * L + l[s]] = e[s];
            l[s] += 1;
            if (moved && !node_ok(x[s], a.num_nodes)) {
                status |= MLXC_STATUS_BAD_NODE;
                stop = true;
            }
            v[s] = x[s];
            if (stop) {
                for (int64_t j = l[s] + 1; j <= L; ++j) out[j] = x[s];
                if (kEdges)
                    for (int64_t j = l[s]; j < L; ++j) a.e_out[n[s] * L + j] = -1;
                l[s] = L;
            }
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------------- uniform walk, windowed

// Per-lane register windows for the two streams of the uniform walk.
//
// The rand stream: walk n reads rand[n*L + l] at step l, so a lane walks
// through its own row 4 bytes at a time while its 63 neighbours do the same
// 4*L bytes apart.  Read one float at a time, nearly every step misses L2 and
// costs a 128-byte line.  Instead each slot keeps the next RW floats of its
// row in registers, loaded as one aligned RW*4-byte block, so the stream
// costs one line per RW steps.
//
// The output: walk n writes n_out[n*(L+1) + j] for j = 0..L, one 8-byte entry
// per step.  Scattered 8-byte stores reach memory as partial 32-byte writes.
// Each slot buffers its entries in an 8-entry window aligned to 64 bytes of
// the output and writes a full window with four 16-byte stores; walks that
// sink in a node of out-degree 0 write their constant tail in whole 64-byte
// blocks.  The stores are non-temporal: the output is never read back, and
// streaming it past the caches keeps them for the graph.
template <int RW>
struct RandWindow {
    float w[RW];
    int valid;  // w[0 .. valid-1] are the next uniforms of the walk
};

template <int RW>
__device__ __forceinline__ void rw_shift1(RandWindow<RW>& r) {
#pragma unroll
    for (int i = 0; i + 1 < RW; ++i) r.w[i] = r.w[i + 1];
}

// Loads the aligned block holding rand[f] and shifts it so w[0] = rand[f].
template <int RW>
__device__ __forceinline__ void rw_load(RandWindow<RW>& r, const float* __restrict__ rand,
                                        int64_t f, int64_t total) {
    const int64_t base = f & ~static_cast<int64_t>(RW - 1);
    if (base + RW <= total) {
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
    } else {  // last block of the array: element loads inside [0, total)
#pragma unroll
        for (int i = 0; i < RW; ++i)
            r.w[i] = (base + i < total) ? __builtin_nontemporal_load(rand + base + i) : 0.0f;
    }
    const int k = static_cast<int>(f - base);
    // shift left by k in log2(RW) conditional steps
#pragma unroll
    for (int bit = RW / 2; bit >= 1; bit >>= 1) {
        if (k & bit) {
#pragma unroll
            for (int i = 0; i < RW; ++i) r.w[i] = (i + bit < RW) ? r.w[i + bit] : 0.0f;
        }
    }
    r.valid = RW - k;
}

// T is the type the entries are buffered in (int32_t when node ids fit);
// they are written as int64.
template <typename T>
struct OutWin {
    T w[8];  // w[8-count .. 7] hold the newest entries; w[7] is entry g
    int count;
};
typedef OutWin<int64_t> OutWindow;

// Writes the buffered entries, the newest of which is output index g.
template <typename T>
__device__ __forceinline__ void ow_flush(OutWin<T>& o, int64_t* __restrict__ out, int64_t g) {
    if (o.count == 8 && ((g + 1) & 7) == 0) {
        int64_t* p = out + (g - 7);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
            i64x2 x = {static_cast<int64_t>(o.w[2 * i]), static_cast<int64_t>(o.w[2 * i + 1])};
            __builtin_nontemporal_store(x, reinterpret_cast<i64x2*>(p + 2 * i));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i >= 8 - o.count)
                __builtin_nontemporal_store(static_cast<int64_t>(o.w[i]), out + g - 7 + i);
    }
    o.count = 0;
}

// Appends the entry for output index g; writes the window when g closes a
// 64-byte block.
template <typename T>
__device__ __forceinline__ void ow_push(OutWin<T>& o, int64_t* __restrict__ out, int64_t g, T x) {
#pragma unroll
    for (int i = 0; i < 7; ++i) o.w[i] = o.w[i + 1];
    o.w[7] = x;
    o.count = o.count < 8 ? o.count + 1 : 8;
    if (((g + 1) & 7) == 0) ow_flush(o, out, g);
}

// Output indices g .. g_last (inclusive) all hold x; the window holds the
// entries before g.  Ends with everything written.
template <typename T>
__device__ __forceinline__ void ow_fill(OutWin<T>& o, int64_t* __restrict__ out, int64_t g,
                                        int64_t g_last, T x) {
    while (g <= g_last && (g & 7) != 0) ow_push(o, out, g++, x);
    if (o.count) ow_flush(o, out, g - 1);
    typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
    const int64_t x64 = static_cast<int64_t>(x);
    const i64x2 xx = {x64, x64};
    for (; g + 7 <= g_last; g += 8) {
        i64x2* p = reinterpret_cast<i64x2*>(out + g);
        __builtin_nontemporal_store(xx, p);
        __builtin_nontemporal_store(xx, p + 1);
        __builtin_nontemporal_store(xx, p + 2);
        __builtin_nontemporal_store(xx, p + 3);
    }
    for (; g <= g_last; ++g) __builtin_nontemporal_store(x64, out + g);
}

// Uniform walk with register windows (requires 16-byte aligned rand and
// n_out; no edge output).  W walk slots per lane, walks from the wave queue.
template <int W, int RW>
__global__ __launch_bounds__(kBlock) void uniform_walk_win_kernel(WalkArgs a) {
    const int64_t L = a.walk_length;
    const int64_t L1 = L + 1;
    const int64_t N = a.num_walks;
    const int64_t rtotal = N * L;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int64_t n[W], v[W], l[W];
    RandWindow<RW> rw[W];
    OutWindow ow[W];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) {
        n[s] = -1;
        l[s] = L;
        v[s] = 0;
        rw[s].valid = 0;
        ow[s].count = 0;
    }

    while (true) {
        bool unretired = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = (n[s] < N) && (l[s] >= L);
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;
                if (id < N) {
                    const int64_t s0 = a.start[id];
                    v[s] = s0;
                    l[s] = 0;
                    rw[s].valid = 0;
                    ow[s].count = 0;
                    ow_push(ow[s], a.n_out, id * L1, s0);
                    if (!node_ok(s0, a.num_nodes)) {
                        status |= MLXC_STATUS_BAD_NODE;
                        ow_fill(ow[s], a.n_out, id * L1 + 1, id * L1 + L, s0);
                        l[s] = L;
                    } else if (L == 0) {
                        ow_flush(ow[s], a.n_out, id * L1);
                    }
                }
            }
            unretired |= (n[s] < N);
        }
        if (!__any(unretired)) break;

        // Phase 1: rowptr pair of every live slot, and a new rand block where
        // the window has run dry.
        RowBounds rb[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            rb[s] = {0, 0};
            if (live) {
                rb[s] = load_row(a.rowptr, v[s]);
                if (rw[s].valid == 0) rw_load(rw[s], a.rand, n[s] * L + l[s], rtotal);
            }
        }
        // Phase 2: candidate edge and its target.
        int64_t x[W];
        bool moved[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            x[s] = v[s];
            moved[s] = false;
            if (live) {
                const int64_t deg = rb[s].end - rb[s].begin;
                if (!row_ok(rb[s], a.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                } else if (deg > 0) {
                    x[s] = a.col[rb[s].begin + pick_index(rw[s].w[0], deg)];
                    moved[s] = true;
                }
            }
        }
        // Phase 3: buffer the new node, advance, finish sunk / broken walks.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            if (!live) continue;
            const int64_t g = n[s] * L1 + l[s] + 1;  // output index of this step
            bool stop = !moved[s];
            if (moved[s] && !node_ok(x[s], a.num_nodes)) {
                status |= MLXC_STATUS_BAD_NODE;
                stop = true;
            }
            v[s] = x[s];
            l[s] += 1;
            rw_shift1(rw[s]);
            rw[s].valid -= 1;
            if (stop) {
                ow_fill(ow[s], a.n_out, g, n[s] * L1 + L, x[s]);
                l[s] = L;
            } else {
                ow_push(ow[s], a.n_out, g, x[s]);
                if (l[s] == L && ow[s].count) ow_flush(ow[s], a.n_out, g);
            }
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------- uniform walk, edge records

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
constexpr size_t kRecordOffset = 256;  // bytes of workspace before the records

__global__ __launch_bounds__(kBlock) void edge_record_kernel(const int64_t* __restrict__ rowptr,
                                                             const int64_t* __restrict__ col,
                                                             int64_t num_nodes, int64_t num_edges,
                                                             EdgeRecord* __restrict__ rec) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < num_edges;
         e += stride) {
        const int64_t c = col[e];
        i32x4 r = {static_cast<int32_t>(c), 0, kRecBadNode, 0};
        if (node_ok(c, num_nodes)) {
            const RowBounds rb = load_row(rowptr, c);
            if (row_ok(rb, num_edges)) {
                r.y = static_cast<int32_t>(rb.begin);
                r.z = static_cast<int32_t>(rb.end - rb.begin);
            } else {
                r.z = kRecBadRow;
            }
        }
        *reinterpret_cast<i32x4*>(rec + e) = r;
    }
}

// Loads the aligned rand block holding rand[f] without shifting it.
template <int RW>
__device__ __forceinline__ void rw_load_block(RandWindow<RW>& r, const float* __restrict__ rand,
                                              int64_t f, int64_t total) {
    const int64_t base = f & ~static_cast<int64_t>(RW - 1);
    if (base + RW <= total) {
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
    } else {
#pragma unroll
        for (int i = 0; i < RW; ++i)
            r.w[i] = (base + i < total) ? __builtin_nontemporal_load(rand + base + i) : 0.0f;
    }
}

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

template <int RW>
__device__ __forceinline__ void rw_shift_by(RandWindow<RW>& r, int k) {
#pragma unroll
    for (int bit = RW / 2; bit >= 1; bit >>= 1) {
        if (k & bit) {
#pragma unroll
            for (int i = 0; i < RW; ++i) r.w[i] = (i + bit < RW) ? r.w[i + bit] : 0.0f;
        }
    }
}

// Start records: walk n's start node in the edge-record format, so a slot
// beginning a walk and a slot taking a step both issue the same single 16-byte
// read.  Written by walk_init_kernel (one coalesced pass over start).
__global__ __launch_bounds__(kBlock) void walk_init_kernel(const int64_t* __restrict__ rowptr,
                                                           const int64_t* __restrict__ start,
                                                           int64_t num_nodes, int64_t num_edges,
                                                           int64_t num_walks,
                                                           EdgeRecord* __restrict__ init) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; n < num_walks;
         n += stride) {
        const int64_t v = start[n];
        i32x4 r = {static_cast<int32_t>(v), 0, kRecBadNode, 0};
        if (node_ok(v, num_nodes)) {
            const RowBounds rb = load_row(rowptr, v);
            if (row_ok(rb, num_edges)) {
                r.y = static_cast<int32_t>(rb.begin);
                r.z = static_cast<int32_t>(rb.end - rb.begin);
            } else {
                r.z = kRecBadRow;
            }
        }
        *reinterpret_cast<i32x4*>(init + n) = r;
    }
}

// Slot phases of the record walk.
enum : int {
    kSlotIdle = 0,   // wants a walk id
    kSlotStart = 1,  // reads the start record of walk n (and its first rand block)
    kSlotWalk = 2,   // reads the record of the chosen edge
    kSlotDone = 3,   // the queue is exhausted
};

// Uniform walk over edge records (requires 16-byte aligned rand and n_out,
// num_nodes and num_edges below 2^31, num_walks * walk_length a multiple of
// 4 and at least RW; no edge output).
//
// Loop invariant: every live slot issues exactly one dependent 16-byte read
// per iteration (a start record or an edge record), plus at most one
// independent rand block, and the wave waits once.  The rand value for a step
// is taken from the window in the iteration before the read it addresses, so
// a new rand block always travels together with a record read and never costs
// a round trip of its own.  Output stores issued after the wait overlap the
// next iteration's read.
template <int W, int RW>
__global__ __launch_bounds__(kBlock) void uniform_walk_rec_kernel(WalkArgs a,
                                                                  const EdgeRecord* __restrict__ recs,
                                                                  const EdgeRecord* __restrict__ init) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int64_t L = a.walk_length;
    const int64_t L1 = L + 1;
    const int64_t N = a.num_walks;
    const int64_t rtotal = N * L;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int phase[W];
    int64_t n[W], l[W], e[W];  // e: record index read this iteration (kSlotWalk)
    int64_t fr[W];             // rand index whose block the next read brings along
    bool need_block[W];        // ... if set
    RandWindow<RW> rw[W];
    OutWin<int32_t> ow[W];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) {
        phase[s] = kSlotIdle;
        n[s] = 0;
        l[s] = 0;
        e[s] = 0;
        fr[s] = 0;
        need_block[s] = false;
        rw[s].valid = 0;
        ow[s].count = 0;
    }

    while (true) {
        // 1. One record read per live slot (idle slots read init[0], so the
        // load is unconditional and nothing merges with it before the wait in
        // step 3), and the rand blocks due.
        int ph[W];  // phase at issue: only these slots consume in step 3
        i32x4 rec[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            ph[s] = phase[s];
            const EdgeRecord* p = ph[s] == kSlotStart ? init + n[s]
                                  : ph[s] == kSlotWalk ? recs + e[s]
                                                       : init;
            rec[s] = *reinterpret_cast<const i32x4*>(p);
        }
#pragma unroll
        for (int s = 0; s < W; ++s)
            if (need_block[s]) rw_load_at(rw[s], a.rand, rw_block_base<RW>(fr[s], rtotal));

        // 2. While the reads are in flight, idle slots draw walk ids from the
        // wave queue; they issue their start reads next iteration.
        bool alive = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = phase[s] == kSlotIdle;
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;
                l[s] = 0;
                phase[s] = id < N ? kSlotStart : kSlotDone;
                fr[s] = id * L;  // the first step's uniform
            }
            alive |= phase[s] != kSlotDone;
        }
        if (!__any(alive)) break;  // every slot done: nothing was read above

        // 3. Consume: buffer the node, finish or pick the next edge.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            if (ph[s] != kSlotStart && ph[s] != kSlotWalk) {
                // a slot that just drew a walk reads its start record and
                // first rand block next iteration
                need_block[s] = phase[s] == kSlotStart && L > 0;
                continue;
            }
            const int64_t g0 = n[s] * L1;  // output index of the walk's start node
            const int64_t g = g0 + l[s] + (ph[s] == kSlotWalk ? 1 : 0);
            if (need_block[s]) {
                // block holding rand[fr]: shift it so w[0] is that value
                const int k = static_cast<int>(fr[s] - rw_block_base<RW>(fr[s], rtotal));
                rw_shift_by(rw[s], k);
                rw[s].valid = RW - k;
                need_block[s] = false;
            }
            const int32_t node = rec[s].x, begin = rec[s].y, deg = rec[s].z;
            bool fill = false, flush = false;
            if (deg < 0) {
                // malformed start or graph entry: stop (outputs unspecified)
                status |= deg == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW;
                if (ph[s] == kSlotStart) ow[s].count = 0;
                ow_fill(ow[s], a.n_out, g, g0 + L, node);
                phase[s] = kSlotIdle;
                continue;
            }
            if (ph[s] == kSlotStart) ow[s].count = 0;
            ow_push(ow[s], a.n_out, g, node);
            if (ph[s] == kSlotWalk) l[s] += 1;
            if (l[s] == L) flush = true;
            else if (deg == 0) fill = true;  // absorbing node: the walk stays
            if (fill) {
                ow_fill(ow[s], a.n_out, g + 1, g0 + L, node);
            } else if (flush) {
                if (ow[s].count) ow_flush(ow[s], a.n_out, g);
            } else {
                // step l (0-based) leaves this node with uniform rand[n*L + l]
                e[s] = begin + pick_index(rw[s].w[0], deg);
                rw_shift1(rw[s]);
                rw[s].valid -= 1;
                need_block[s] = rw[s].valid == 0 && l[s] + 1 < L;
                fr[s] = n[s] * L + l[s] + 1;
                phase[s] = kSlotWalk;
            }
            if (fill || flush) phase[s] = kSlotIdle;
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// ---------------------------------------------------------- node2vec walk

struct N2VArgs {
    WalkArgs w;
    double prob0, prob1, prob2;
    uint32_t key0, key1;
};

// Is t in row(x)?  BiasedRandomWalk.cpp:20-28 scans the row linearly; on a
// sorted row lower_bound gives the same answer in log2(deg) probes.
template <bool kSorted>
__device__ __forceinline__ bool is_neighbor(const int64_t* __restrict__ rowptr,
                                            const int64_t* __restrict__ col, int64_t num_edges,
                                            int64_t x, int64_t t, uint32_t& status) {
    const RowBounds rb = load_row(rowptr, x);
    if (!row_ok(rb, num_edges)) {
        status |= MLXC_STATUS_BAD_ROW;
        return false;
    }
    if (!kSorted) {
        for (int64_t i = rb.begin; i < rb.end; ++i)
            if (col[i] == t) return true;
        return false;
    }
    int64_t lo = rb.begin, count = rb.end - rb.begin;
    while (count > 0) {
        const int64_t half = count >> 1;
        const int64_t mid = lo + half;
        if (col[mid] < t) {
            lo = mid + 1;
            count -= half + 1;
        } else {
            count = half;
        }
    }
    return lo < rb.end && col[lo] == t;
}

// Acceptance of candidate x after previous node t (see accept rules in
// mlxc.h).  The reference's chain (BiasedRandomWalk.cpp:86-91) has no side
// effects, so the row search runs only when its answer decides the result.
template <int kRule, bool kSorted>
__device__ __forceinline__ bool accept(const N2VArgs& a, double r, int64_t x, int64_t t,
                                       uint32_t& status) {
    if (kRule == MLXC_RULE_REF_CHAIN) {
        if (r < a.prob2) return true;
        if (x == t && r < a.prob0) return true;
        if (r < a.prob1)
            return is_neighbor<kSorted>(a.w.rowptr, a.w.col, a.w.num_edges, x, t, status);
        return false;
    }
    if (x == t) return r < a.prob0;
    const bool lt1 = r < a.prob1, lt2 = r < a.prob2;
    if (lt1 && lt2) return true;
    if (!lt1 && !lt2) return false;
    return is_neighbor<kSorted>(a.w.rowptr, a.w.col, a.w.num_edges, x, t, status) ? lt1 : lt2;
}

template <int kRule, bool kSorted, bool kEdges>
__global__ __launch_bounds__(kBlock) void node2vec_walk_kernel(N2VArgs a) {
    const int64_t L = a.w.walk_length;
    const int64_t N = a.w.num_walks;
    const int64_t V = a.w.num_nodes;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.w.work + 1);
    WaveQueue q{0, 0};
    uint32_t status = 0;
    while (true) {
        const int64_t n = queue_take(q, true, counter);
        if (n >= N) break;  // wave-uniform: every lane asked, ids are consecutive
        int64_t* out = a.w.n_out + n * (L + 1);
        int64_t* eout = kEdges ? a.w.e_out + n * L : nullptr;
        int64_t t = a.w.start[n];
        out[0] = t;
        if (L == 0) {
            if (!node_ok(t, V)) status |= MLXC_STATUS_BAD_NODE;
            continue;
        }
        bool bad = !node_ok(t, V);
        int64_t v = t, e = -1;
        const uint32_t n_lo = static_cast<uint32_t>(n), n_hi = static_cast<uint32_t>(n >> 32);
        if (bad) {
            status |= MLXC_STATUS_BAD_NODE;
        } else {
            // First step: uniform, no acceptance test (BiasedRandomWalk.cpp:60-66).
            const RowBounds rb = load_row(a.w.rowptr, t);
            if (!row_ok(rb, a.w.num_edges)) {
                status |= MLXC_STATUS_BAD_ROW;
                bad = true;
            } else if (rb.end > rb.begin) {
                uint32_t c0 = n_lo, c1 = n_hi, c2 = 0, c3 = 0;
                philox4x32_10(c0, c1, c2, c3, a.key0, a.key1);
                e = rb.begin + pick_index(unit_float(c0), rb.end - rb.begin);
                v = a.w.col[e];
            }
        }
        out[1] = v;
        if (kEdges) eout[0] = e;
        for (int64_t l = 1; l < L; ++l) {
            int64_t x = v;
            e = -1;
            if (!bad && !node_ok(v, V)) {
                status |= MLXC_STATUS_BAD_NODE;
                bad = true;
            }
            if (!bad) {
                const RowBounds rb = load_row(a.w.rowptr, v);
                const int64_t deg = rb.end - rb.begin;
                if (!row_ok(rb, a.w.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                    bad = true;
                } else if (deg == 1) {  // BiasedRandomWalk.cpp:76-78: forced, no draw
                    e = rb.begin;
                    x = a.w.col[e];
                } else if (deg > 1) {   // :80-92 rejection loop
                    for (uint32_t trial = 0;; ++trial) {
                        uint32_t c0 = n_lo, c1 = n_hi, c2 = static_cast<uint32_t>(l), c3 = trial;
                        philox4x32_10(c0, c1, c2, c3, a.key0, a.key1);
                        e = rb.begin + pick_index(unit_float(c0), deg);
                        x = a.w.col[e];
                        const double r = static_cast<double>(unit_float(c1));
                        if (!node_ok(x, V)) {
                            status |= MLXC_STATUS_BAD_NODE;
                            bad = true;
                            break;
                        }
                        if (accept<kRule, kSorted>(a, r, x, t, status)) break;
                        if (trial + 1 >= MLXC_MAX_TRIALS) break;
                    }
                }
            }
            out[l + 1] = x;
            if (kEdges) eout[l] = e;
            t = v;
            v = x;
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------------------------- CSR check

__device__ __forceinline__ int64_t wave_sum(int64_t x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

// work[0] |= MLXC_CSR_BAD_ROWPTR / MLXC_CSR_BAD_COL bits; work[1] counts
// positions i >= 1 with col[i] < col[i-1]; work[2] counts those positions
// that start a non-empty row.  Rows are sorted iff work[1] == work[2].
__global__ __launch_bounds__(kBlock) void csr_check_kernel(const int64_t* __restrict__ rowptr,
                                                           int64_t V,
                                                           const int64_t* __restrict__ col,
                                                           int64_t E, int64_t* work) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    uint32_t bits = 0;
    int64_t desc = 0, start_desc = 0;
    if (gid == 0 && (rowptr[0] != 0 || rowptr[V] != E)) bits |= MLXC_CSR_BAD_ROWPTR;
    for (int64_t v = gid; v < V; v += stride) {
        const int64_t rs = rowptr[v], re = rowptr[v + 1];
        if (re < rs) bits |= MLXC_CSR_BAD_ROWPTR;
        if (rs >= 1 && re > rs && re <= E && col[rs] < col[rs - 1]) ++start_desc;
    }
    for (int64_t i = gid; i < E; i += stride) {
        const int64_t c = col[i];
        if (!node_ok(c, V)) bits |= MLXC_CSR_BAD_COL;
        if (i >= 1 && c < col[i - 1]) ++desc;
    }
    const int64_t d = wave_sum(desc), sd = wave_sum(start_desc);
    const uint64_t any_bits = __ballot(bits != 0);
    uint32_t wave_bits = bits;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) wave_bits |= __shfl_xor(wave_bits, off, kWave);
    if (__lane_id() == 0) {
        if (any_bits) atomicOr(reinterpret_cast<unsigned long long*>(work), static_cast<unsigned long long>(wave_bits));
        if (d) atomicAdd(reinterpret_cast<unsigned long long*>(work + 1), static_cast<unsigned long long>(d));
        if (sd) atomicAdd(reinterpret_cast<unsigned long long*>(work + 2), static_cast<unsigned long long>(sd));
    }
}

// ----------------------------------------------------------- Philox fill

__global__ __launch_bounds__(kBlock) void philox_fill_kernel(float* __restrict__ out, int64_t n,
                                                             uint32_t k0, uint32_t k1) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t blocks = (n + 3) >> 2;
    for (int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; j < blocks; j += stride) {
        uint32_t c0 = static_cast<uint32_t>(j), c1 = static_cast<uint32_t>(static_cast<uint64_t>(j) >> 32);
        uint32_t c2 = 0, c3 = 0;
        philox4x32_10(c0, c1, c2, c3, k0, k1);
        const int64_t i = j << 2;
        if (i + 3 < n) {
            out[i] = unit_float(c0);
            out[i + 1] = unit_float(c1);
            out[i + 2] = unit_float(c2);
            out[i + 3] = unit_float(c3);
        } else {
            const uint32_t w[4] = {c0, c1, c2, c3};
            for (int k = 0; k < 4 && i + k < n; ++k) out[i + k] = unit_float(w[k]);
        }
    }
}

// ------------------------------------------------------------ launch help

struct DeviceInfo {
    int cus = 0;
};

int device_info(DeviceInfo& info) {
    static std::mutex mu;
    static DeviceInfo cache[64];
    int dev = 0;
    MLXC_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(MLXC_ERR_HIP, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (cache[dev].cus == 0) {
        int cus = 0;
        MLXC_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        cache[dev].cus = cus;
    }
    info = cache[dev];
    return MLXC_OK;
}

// Persistent grid: the blocks that stay resident on the device, but no
// more than the walks can feed (each block serves W * kBlock walks at once).
template <typename Kernel>
int persistent_grid(Kernel kernel, int64_t num_walks, int walks_per_lane, int& grid) {
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    int per_cu = 0;
    MLXC_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kBlock, 0));
    if (per_cu < 1) per_cu = 1;
    const int64_t resident = static_cast<int64_t>(info.cus) * per_cu;
    const int64_t per_block = static_cast<int64_t>(walks_per_lane) * kBlock;
    const int64_t feedable = (num_walks + per_block - 1) / per_block;
    grid = static_cast<int>(feedable < resident ? feedable : resident);
    if (grid < 1) grid = 1;
    return MLXC_OK;
}

int check_common(const int64_t* rowptr, int64_t num_nodes, const int64_t* col, int64_t num_edges,
                 const int64_t* start, int64_t num_walks, int32_t walk_length,
                 const int64_t* n_out, const void* work, size_t work_bytes) {
    if (num_nodes < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes must be >= 0");
    if (num_edges < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_edges must be >= 0");
    if (num_walks < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_walks must be >= 0");
    if (walk_length < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "walk_length must be >= 0");
    if (!work) return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must not be NULL");
    if (work_bytes < MLXC_WORK_WORDS * sizeof(int64_t))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must hold at least MLXC_WORK_WORDS int64 words");
    if (reinterpret_cast<uintptr_t>(work) % 16 != 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    if (num_walks > 0) {
        if (!rowptr || !start || !n_out)
            return fail(MLXC_ERR_INVALID_ARGUMENT, "rowptr, start and n_out must not be NULL");
        if (num_edges > 0 && !col) return fail(MLXC_ERR_INVALID_ARGUMENT, "col must not be NULL");
        if (num_walks > INT64_MAX / (static_cast<int64_t>(walk_length) + 1))
            return fail(MLXC_ERR_INVALID_ARGUMENT, "num_walks * (walk_length + 1) overflows int64");
    }
    return MLXC_OK;
}

int zero_work(int64_t* d_work, hipStream_t stream) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kWave), 0, stream, d_work, MLXC_WORK_WORDS);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

#ifndef MLXC_UNIFORM_SLOTS
#define MLXC_UNIFORM_SLOTS 1   // walks in flight per lane
#endif
#ifndef MLXC_RAND_WINDOW
#define MLXC_RAND_WINDOW 16    // uniforms per rand block (4-byte floats)
#endif

template <typename Kernel>
int launch_persistent(Kernel kernel, const WalkArgs& a, int slots, hipStream_t stream) {
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.num_walks, slots, grid)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

bool records_fit(int64_t num_nodes, int64_t num_edges) {
    return num_nodes <= INT32_MAX && num_edges <= INT32_MAX;
}

size_t record_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks) {
    if (!records_fit(num_nodes, num_edges) || num_walks < 0)
        return MLXC_WORK_WORDS * sizeof(int64_t);
    return kRecordOffset + static_cast<size_t>(num_edges + num_walks) * sizeof(EdgeRecord);
}

int launch_uniform(const WalkArgs& a, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
    constexpr int W = MLXC_UNIFORM_SLOTS;
    const bool aligned = (reinterpret_cast<uintptr_t>(a.rand) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(a.n_out) % 16 == 0);
    if (a.e_out) return launch_persistent(uniform_walk_kernel<W, true>, a, W, stream);
    if (!aligned) return launch_persistent(uniform_walk_kernel<W, false>, a, W, stream);
    const int64_t rtotal = a.num_walks * a.walk_length;
    if (records_fit(a.num_nodes, a.num_edges) && rtotal % 4 == 0 && rtotal >= MLXC_RAND_WINDOW &&
        workspace_bytes >= record_workspace_bytes(a.num_nodes, a.num_edges, a.num_walks)) {
        EdgeRecord* recs = reinterpret_cast<EdgeRecord*>(static_cast<char*>(workspace) + kRecordOffset);
        EdgeRecord* init = recs + a.num_edges;
        DeviceInfo info;
        if (int rc = device_info(info)) return rc;
        const int64_t cap = static_cast<int64_t>(info.cus) * 16;
        if (a.num_edges > 0) {
            int64_t grid = (a.num_edges + kBlock - 1) / kBlock;
            if (grid > cap) grid = cap;
            hipLaunchKernelGGL(edge_record_kernel, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0,
                               stream, a.rowptr, a.col, a.num_nodes, a.num_edges, recs);
            MLXC_HIP_TRY(hipGetLastError());
        }
        int64_t igrid = (a.num_walks + kBlock - 1) / kBlock;
        if (igrid > cap) igrid = cap;
        hipLaunchKernelGGL(walk_init_kernel, dim3(static_cast<unsigned>(igrid)), dim3(kBlock), 0,
                           stream, a.rowptr, a.start, a.num_nodes, a.num_edges, a.num_walks, init);
        MLXC_HIP_TRY(hipGetLastError());
        auto kernel = uniform_walk_rec_kernel<W, MLXC_RAND_WINDOW>;
        int grid = 0;
        if (int rc = persistent_grid(kernel, a.num_walks, W, grid)) return rc;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a,
                           static_cast<const EdgeRecord*>(recs), static_cast<const EdgeRecord*>(init));
        MLXC_HIP_TRY(hipGetLastError());
        return MLXC_OK;
    }
    return launch_persistent(uniform_walk_win_kernel<W, MLXC_RAND_WINDOW>, a, W, stream);
}

template <int kRule, bool kSorted, bool kEdges>
int launch_node2vec(const N2VArgs& a, hipStream_t stream) {
    auto kernel = node2vec_walk_kernel<kRule, kSorted, kEdges>;
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

template <int kRule>
int dispatch_node2vec(const N2VArgs& a, bool sorted, bool edges, hipStream_t stream) {
    if (sorted)
        return edges ? launch_node2vec<kRule, true, true>(a, stream)
                     : launch_node2vec<kRule, true, false>(a, stream);
    return edges ? launch_node2vec<kRule, false, true>(a, stream)
                 : launch_node2vec<kRule, false, false>(a, stream);
}

}  // namespace

// =================================================================== C ABI

extern "C" {

int mlxc_version(void) { return 100; }

const char* mlxc_last_error(void) { return g_last_error.c_str(); }

size_t mlxc_walk_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks) {
    if (num_nodes < 0 || num_edges < 0) return MLXC_WORK_WORDS * sizeof(int64_t);
    return record_workspace_bytes(num_nodes, num_edges, num_walks);
}

int mlxc_random_walk(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                     int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                     const float* d_rand, int32_t walk_length, int64_t* d_n_out,
                     int64_t* d_e_out, void* d_workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_common(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                              walk_length, d_n_out, d_workspace, workspace_bytes))
        return rc;
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (num_walks > 0 && walk_length > 0 && !d_rand)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "rand must not be NULL");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = zero_work(d_work, s)) return rc;
    if (num_walks == 0) return MLXC_OK;
    WalkArgs a{d_rowptr, d_col, d_start, d_rand, d_n_out, d_e_out, d_work,
               num_nodes, num_edges, num_walks, walk_length};
    return launch_uniform(a, d_workspace, workspace_bytes, s);
}

int mlxc_rejection_sampling(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                            int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                            int32_t walk_length, double p, double q, uint64_t seed,
                            int32_t rule, int32_t rows_sorted, int64_t* d_n_out,
                            int64_t* d_e_out, void* d_workspace, size_t workspace_bytes,
                            void* stream) {
    if (int rc = check_common(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                              walk_length, d_n_out, d_workspace, workspace_bytes))
        return rc;
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (!(p > 0.0) || !(q > 0.0) || !std::isfinite(p) || !std::isfinite(q))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "p and q must be finite and > 0");
    if (rule != MLXC_RULE_REF_CHAIN && rule != MLXC_RULE_NODE2VEC_EXACT)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "rule must be MLXC_RULE_REF_CHAIN or MLXC_RULE_NODE2VEC_EXACT");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = zero_work(d_work, s)) return rc;
    if (num_walks == 0) return MLXC_OK;
    // Acceptance constants exactly as BiasedRandomWalk.cpp:52-55, in FP64.
    const double max_prob = std::fmax(std::fmax(1. / p, 1.), 1. / q);
    N2VArgs a;
    a.w = WalkArgs{d_rowptr, d_col, d_start, nullptr, d_n_out, d_e_out, d_work,
                   num_nodes, num_edges, num_walks, walk_length};
    a.prob0 = 1. / p / max_prob;
    a.prob1 = 1. / max_prob;
    a.prob2 = 1. / q / max_prob;
    a.key0 = static_cast<uint32_t>(seed);
    a.key1 = static_cast<uint32_t>(seed >> 32);
    const bool sorted = rows_sorted != 0, edges = d_e_out != nullptr;
    return rule == MLXC_RULE_REF_CHAIN
               ? dispatch_node2vec<MLXC_RULE_REF_CHAIN>(a, sorted, edges, s)
               : dispatch_node2vec<MLXC_RULE_NODE2VEC_EXACT>(a, sorted, edges, s);
}

int mlxc_csr_check(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                   int64_t num_edges, void* d_workspace, size_t workspace_bytes, int32_t* h_flags,
                   void* stream) {
    if (num_nodes < 0 || num_edges < 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes and num_edges must be >= 0");
    if (!d_rowptr || !d_workspace || !h_flags || (num_edges > 0 && !d_col))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "NULL pointer argument");
    if (workspace_bytes < MLXC_WORK_WORDS * sizeof(int64_t))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must hold at least MLXC_WORK_WORDS int64 words");
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = zero_work(d_work, s)) return rc;
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    const int64_t items = num_nodes > num_edges ? num_nodes : num_edges;
    int64_t grid = (items + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(info.cus) * 8;
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(csr_check_kernel, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, s,
                       d_rowptr, num_nodes, d_col, num_edges, d_work);
    MLXC_HIP_TRY(hipGetLastError());
    int64_t host[3] = {0, 0, 0};
    MLXC_HIP_TRY(hipMemcpyAsync(host, d_work, sizeof(host), hipMemcpyDeviceToHost, s));
    MLXC_HIP_TRY(hipStreamSynchronize(s));
    int32_t flags = static_cast<int32_t>(host[0]);
    if (!(flags & MLXC_CSR_BAD_ROWPTR) && host[1] != host[2]) flags |= MLXC_CSR_UNSORTED;
    *h_flags = flags;
    return MLXC_OK;
}

int mlxc_philox_uniform(float* d_out, int64_t n, uint64_t seed, void* stream) {
    if (n < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n == 0) return MLXC_OK;
    if (!d_out) return fail(MLXC_ERR_INVALID_ARGUMENT, "out must not be NULL");
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    const int64_t blocks4 = (n + 3) / 4;
    int64_t grid = (blocks4 + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(info.cus) * 16;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(philox_fill_kernel, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), d_out, n, static_cast<uint32_t>(seed),
                       static_cast<uint32_t>(seed >> 32));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

}  // extern "C"
