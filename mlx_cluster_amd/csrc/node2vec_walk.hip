// node2vec walk by rejection sampling (BiasedRandomWalk.cpp:52-100) and its
// launcher.  The reference has no GPU version (BiasedRandomWalk.cpp:150-155).
#include <cmath>
#include <limits>

#include "walk_host.h"

namespace mlxc {

struct N2VArgs {
    WalkArgs w;
    double prob0, prob1, prob2;
    uint32_t key0, key1;
    int32_t rows;  // MLXC_ROWS_*; DETECT: work[2] != 0 when the rows are sorted
};

// Entries per round of the direct kernel's scan of an unsorted row (one
// 128-byte line of int64).  Configuration 3's graph with every row scanned
// (2^18 walks of 10 steps) on MI355X: 152, 112 and 104 ms with rounds of 4,
// 8 and 16 entries, 256 ms one entry at a time.
#ifndef MLXC_SCAN_ROUND
#define MLXC_SCAN_ROUND 16
#endif
constexpr int kScanRound = MLXC_SCAN_ROUND;

// Is t in row(x)?  BiasedRandomWalk.cpp:20-28 scans the row linearly; on a
// sorted row lower_bound gives the same answer in log2(deg) probes.
__device__ __forceinline__ bool is_neighbor(const int64_t* __restrict__ rowptr,
                                            const int64_t* __restrict__ col, int64_t num_edges,
                                            bool sorted, int64_t x, int64_t t, uint32_t& status) {
    const RowBounds rb = load_row(rowptr, x);
    if (!row_ok(rb, num_edges)) {
        status |= MLXC_STATUS_BAD_ROW;
        return false;
    }
    if (!sorted) {
        // kScanRound entries per round, loaded unconditionally (indices past
        // the row's end are clamped to its last entry): the loads are
        // independent, so a round costs one memory round trip, where one
        // entry at a time waits for each load
        for (int64_t i = rb.begin; i < rb.end; i += kScanRound) {
            int64_t v[kScanRound];
#pragma unroll
            for (int k = 0; k < kScanRound; ++k) v[k] = col[i + k < rb.end ? i + k : rb.end - 1];
            bool hit = false;
#pragma unroll
            for (int k = 0; k < kScanRound; ++k) hit |= v[k] == t;  // (a clamped entry repeats one in the row)
            if (hit) return true;
        }
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
template <int kRule>
__device__ __forceinline__ bool accept(const N2VArgs& a, bool sorted, double r, int64_t x,
                                       int64_t t, uint32_t& status) {
    if (kRule == MLXC_RULE_REF_CHAIN) {
        if (r < a.prob2) return true;
        if (x == t && r < a.prob0) return true;
        if (r < a.prob1)
            return is_neighbor(a.w.rowptr, a.w.col, a.w.num_edges, sorted, x, t, status);
        return false;
    }
    if (x == t) return r < a.prob0;
    const bool lt1 = r < a.prob1, lt2 = r < a.prob2;
    if (lt1 && lt2) return true;
    if (!lt1 && !lt2) return false;
    return is_neighbor(a.w.rowptr, a.w.col, a.w.num_edges, sorted, x, t, status) ? lt1 : lt2;
}

// node2vec walk on the CSR arrays (the fallback of the record walk, and the
// walk of graphs whose ids exceed int32).  The row order comes from the
// device: csr_status_kernel leaves work[2] = 1 when the CSR check found every
// row sorted, so the call needs no host round trip.
//
// Each lane takes its own walks from the wave queue and does one trial of
// its current step per loop iteration (reading the step's row first when it
// enters the step), so lanes never wait for each other's rejection runs or
// walk ends.  A walk that meets an out-of-range id or row, or a node of
// out-degree 0, repeats its node to the end: a bad candidate id is written
// once, then repeated.
template <int kRule, bool kEdges, typename OutT>
__global__ __launch_bounds__(kBlock) void node2vec_walk_kernel(N2VArgs a) {
    const int64_t L = a.w.walk_length;
    const int64_t N = a.w.num_walks;
    const int64_t V = a.w.num_nodes;
    const bool sorted = a.rows == MLXC_ROWS_SORTED ||
                        (a.rows == MLXC_ROWS_DETECT && a.w.work[2] != 0);
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.w.work + 1);
    WaveQueue q{0, 0};
    uint32_t status = 0;
    OutT* out = nullptr;
    OutT* eout = nullptr;
    int64_t n = 0, l = 0;     // walk and its step (1 .. L-1 while walking)
    int64_t t = 0, v = 0;     // previous and current node
    RowBounds rb{0, 0};       // row of v, once the step has been entered
    uint32_t n_lo = 0, n_hi = 0, trial = 0;
    bool walking = false;     // walk n has step l to take
    bool entered = false;     // ... and has read v's row (rb)
    bool exhausted = false;   // the queue has no walk left for this lane
    // steps l .. L-1 stay at node x with no edge
    auto stay = [&](int64_t from, int64_t x) {
        for (int64_t j = from; j < L; ++j) {
            out[j + 1] = static_cast<OutT>(x);
            if (kEdges) eout[j] = static_cast<OutT>(-1);
        }
        walking = false;
    };
    while (true) {
        const bool need = !walking && !exhausted;
        const int64_t id = queue_take(q, need, counter);
        if (need) {
            if (id >= N) {
                exhausted = true;
            } else {
                n = id;
                const int64_t sn = a.w.walk_base + n;  // the walk's Philox stream index
                n_lo = static_cast<uint32_t>(sn);
                n_hi = static_cast<uint32_t>(sn >> 32);
                out = static_cast<OutT*>(a.w.n_out) + n * (L + 1);
                eout = kEdges ? static_cast<OutT*>(a.w.e_out) + n * L : nullptr;
                t = a.w.start[n];
                out[0] = static_cast<OutT>(t);
                if (L == 0) {
                    if (!node_ok(t, V)) status |= MLXC_STATUS_BAD_NODE;
                } else {
                    // first step: uniform, no acceptance test (BiasedRandomWalk.cpp:60-66)
                    bool bad = !node_ok(t, V);
                    int64_t e = -1;
                    v = t;
                    if (bad) {
                        status |= MLXC_STATUS_BAD_NODE;
                    } else {
                        const RowBounds r0 = load_row(a.w.rowptr, t);
                        if (!row_ok(r0, a.w.num_edges)) {
                            status |= MLXC_STATUS_BAD_ROW;
                            bad = true;
                        } else if (r0.end > r0.begin) {
                            uint32_t c0 = n_lo, c1 = n_hi, c2 = 0, c3 = 0;
                            philox4x32_10(c0, c1, c2, c3, a.key0, a.key1);
                            e = r0.begin + pick_index(unit_float(c0), r0.end - r0.begin);
                            v = a.w.col[e];
                        }
                    }
                    out[1] = static_cast<OutT>(v);
                    if (kEdges) eout[0] = static_cast<OutT>(e);
                    l = 1;
                    walking = true;
                    entered = false;
                    if (bad) stay(1, v);
                    else if (L == 1) walking = false;
                }
            }
        }
        if (!__any(walking || !exhausted)) break;
        if (!walking) continue;
        if (!entered) {
            if (!node_ok(v, V)) {
                status |= MLXC_STATUS_BAD_NODE;
                stay(l, v);
                continue;
            }
            rb = load_row(a.w.rowptr, v);
            const int64_t deg = rb.end - rb.begin;
            if (!row_ok(rb, a.w.num_edges)) {
                status |= MLXC_STATUS_BAD_ROW;
                stay(l, v);
                continue;
            }
            if (deg == 0) {
                stay(l, v);  // an absorbing node: the walk stays
                continue;
            }
            entered = true;
            trial = 0;
        }
        const int64_t deg = rb.end - rb.begin;
        int64_t e, x;
        bool take;
        if (deg == 1) {  // BiasedRandomWalk.cpp:76-78: forced, no draw
            e = rb.begin;
            x = a.w.col[e];
            take = true;
        } else {         // :80-92, one trial of the rejection loop
            uint32_t c0 = n_lo, c1 = n_hi, c2 = static_cast<uint32_t>(l), c3 = trial;
            philox4x32_10(c0, c1, c2, c3, a.key0, a.key1);
            e = rb.begin + pick_index(unit_float(c0), deg);
            x = a.w.col[e];
            const double r = static_cast<double>(unit_float(c1));
            if (!node_ok(x, V)) {
                status |= MLXC_STATUS_BAD_NODE;
                out[l + 1] = static_cast<OutT>(x);
                if (kEdges) eout[l] = static_cast<OutT>(e);
                stay(l + 1, x);
                continue;
            }
            take = accept<kRule>(a, sorted, r, x, t, status) || trial + 1 >= MLXC_MAX_TRIALS;
        }
        if (!take) {
            ++trial;
            continue;
        }
        out[l + 1] = static_cast<OutT>(x);
        if (kEdges) eout[l] = static_cast<OutT>(e);
        t = v;
        v = x;
        ++l;
        entered = false;
        if (l == L) walking = false;
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// ---------------------------------------------------- record node2vec walk

// Slot phases of the record walk.
enum : int {
    kN2vIdle = 0,    // wants a walk id
    kN2vStart = 1,   // reads the start record of walk n
    kN2vCand = 2,    // reads the edge record of the current candidate
    kN2vLevel = 3,   // sorted rows: reads one 16-entry block of a search-index level
    kN2vScan = 4,    // unsorted rows: reads the next 16 entries of row(x)
    kN2vDone = 5,    // the queue is exhausted
    kN2vRow = 6,     // CSR mode: reads rowptr[x], rowptr[x + 1] of the candidate
    kN2vBit = 7,     // reads the word of a hub bitmap that answers the neighbour test
    kN2vHash = 8,    // reads one bucket of a row hash table
};

// What a CSR-mode slot does once the candidate's row has been read.
enum : int {
    kRowAccept = 0,  // take the step
    kRowSearch = 1,  // search t in row(x), then decide
};

// The two uniforms of a trial: Philox4x32-10 with key = seed and counter =
// (walk lo, walk hi, step, trial), walk being the stream index walk_base + n
// of walk n of the call; word 0 picks the candidate, word 1 is
// the acceptance test's r (the reference's rand() % deg and rand()/RAND_MAX,
// BiasedRandomWalk.cpp:81,84).
__device__ __forceinline__ void n2v_uniforms(int64_t n, int32_t step, uint32_t trial,
                                             uint32_t k0, uint32_t k1, float& u0, float& u1) {
    uint32_t c0 = static_cast<uint32_t>(n), c1 = static_cast<uint32_t>(static_cast<uint64_t>(n) >> 32);
    uint32_t c2 = static_cast<uint32_t>(step), c3 = trial;
    philox4x32_10(c0, c1, c2, c3, k0, k1);
    u0 = unit_float(c0);
    u1 = unit_float(c1);
}

// Neighbour search on sorted rows, through the levels of IndexLevels.  Inside
// a sorted row the level-k samples are sorted too, so one aligned block of 16
// level-k entries splits the 16^(k+1) col32 positions it covers into 16
// segments of 16^k positions: one read narrows the search to one segment,
// which is exactly one aligned block of level k-1.  A search for t in row
// [b, e) starts at the finest level at which one block covers the whole row
// and ends with one 64-byte block of col32: k + 1 dependent reads for a row
// of up to 16^(k+1) entries, from arrays 16 times smaller per level (the
// upper levels stay in L2).  Bisection needs about log2(deg / 16) reads of
// the E/16-entry level instead.
//
// lo, hi: the col32 positions that can still hold t.  Returns 1 (found), 0
// (absent) or -1 (continue with the updated lvl, blk, lo, hi).
__device__ __forceinline__ int level_step(const int32_t (&v)[kSearchBlock], int32_t t, int& lvl,
                                          int32_t& blk, int32_t& lo, int32_t& hi) {
    const int sh = 4 * lvl;  // log2 of the distance S between samples of this level
    const int64_t base = static_cast<int64_t>(kSearchBlock) * blk << sh;  // sample 0's position
    // samples i_lo .. i_hi-1 of the block lie in [lo, hi): ceil((lo - base) / S) ..
    const int64_t s_minus_1 = (int64_t{1} << sh) - 1;
    const int i_lo = lo > base ? static_cast<int>(min(int64_t{kSearchBlock}, (lo - base + s_minus_1) >> sh)) : 0;
    const int i_hi = hi > base ? static_cast<int>(min(int64_t{kSearchBlock}, (hi - base + s_minus_1) >> sh)) : 0;
    int best = -1;       // last sample in [lo, hi) that is <= t
    bool found = false;  // a sample in [lo, hi) equals t
#pragma unroll
    for (int i = 0; i < kSearchBlock; ++i) {
        const bool inside = i >= i_lo && i < i_hi;
        if (inside && v[i] <= t) best = i;
        found |= inside && v[i] == t;
    }
    if (found) return 1;
    if (lvl == 0) return 0;
    if (best >= 0) {
        // t is after sample best and before the next one: the segment
        // [pos, pos + S) is block kSearchBlock * blk + best of level lvl-1
        const int64_t pos = base + (static_cast<int64_t>(best) << sh);
        lo = static_cast<int32_t>(pos + 1);
        hi = static_cast<int32_t>(min(static_cast<int64_t>(hi), pos + s_minus_1 + 1));
        blk = kSearchBlock * blk + best;
    } else {
        // every sample of the row here is > t: t is before the first one
        hi = static_cast<int32_t>(min(static_cast<int64_t>(hi), base + (static_cast<int64_t>(i_lo) << sh)));
        blk = static_cast<int32_t>(static_cast<int64_t>(lo) >> sh);
    }
    lvl -= 1;
    return lo < hi ? -1 : 0;
}

// Linear scan of an unsorted row, 16 entries (one 64-byte block of col32)
// per read: the entries of block lo / 16 inside [lo, hi).
__device__ __forceinline__ int scan_step(const int32_t (&v)[kSearchBlock], int32_t t, int32_t& lo,
                                         int32_t hi) {
    const int32_t base = lo & ~(kSearchBlock - 1);
    bool found = false;
#pragma unroll
    for (int i = 0; i < kSearchBlock; ++i) {
        const int32_t pos = base + i;
        found |= pos >= lo && pos < hi && v[i] == t;
    }
    if (found) return 1;
    lo = base + kSearchBlock;
    return lo < hi ? -1 : 0;
}

struct N2VRecArgs {
    WalkArgs w;
    const EdgeRecord* recs;   // [num_edges]; null in CSR mode
    const EdgeRecord* init;   // [num_walks]
    IndexLevels index;        // search index (level 0 = col32)
    int32_t rows;             // MLXC_ROWS_*; DETECT reads the prep pass's counts in work[2..3]
    int32_t symmetric;        // the graph is symmetric: search the shorter row
    // The acceptance probabilities as the smallest floats >= prob0, prob1,
    // prob2: for a float r, r < prob_k (in double, as the reference compares)
    // exactly when r < thr_k.
    float thr0, thr1, thr2;
    uint32_t key0, key1;
    // Hub bitmaps (record mode; null: none): bitmap s is hub_words words from
    // hub_bits + s * hub_words, and the records carry each node's slot.
    const uint32_t* hub_bits;
    int64_t hub_words;
    const int32_t* row32;  // int32 row starts (row32_kernel): the CSR mode's row reads
    // Row hash tables (record mode; null: none), kSearchBlock slots a bucket:
    // rows without a hub bitmap whose search would take more than one read.
    const int32_t* hash;
    // LDS walk: the walks a block runs at once (all its threads copy the
    // graph), and the lanes that run each walk (1, 2, 4, 8 or 16)
    int32_t lds_walkers;
    int32_t lds_group;
    // record walk: walks per wavefront of a call of few walks, which skips
    // the queue and runs them all in the tail phase (0: the queue)
    int32_t tail_direct;
};

// Smallest float >= p (p > 0), the float threshold of N2VRecArgs.
static float float_at_or_above(double p) {
    float f = static_cast<float>(p);
    if (static_cast<double>(f) < p) f = std::nextafter(f, std::numeric_limits<float>::infinity());
    return f;
}

// Decision on candidate x for r before any row search: 1 accept, 0 reject,
// -1 the answer depends on whether t is in row(x).  The reference's chain
// (BiasedRandomWalk.cpp:86-91: (x==t && r<p0) || (nb(x,t) && r<p1) || r<p2)
// has no side effects, so its cheap terms decide first; the analytic rule
// uses p0 when x == t, else p1 or p2 by adjacency.
template <int kRule>
__device__ __forceinline__ int n2v_decide(const N2VRecArgs& a, float r, int32_t x, int32_t t) {
    if (kRule == MLXC_RULE_REF_CHAIN) {
        if (r < a.thr2) return 1;
        if (x == t && r < a.thr0) return 1;
        return r < a.thr1 ? -1 : 0;
    }
    if (x == t) return r < a.thr0 ? 1 : 0;
    const bool lt1 = r < a.thr1, lt2 = r < a.thr2;
    if (lt1 && lt2) return 1;
    if (!lt1 && !lt2) return 0;
    return -1;
}

// The row the neighbour test searches: t in row(x), as the reference does
// (BiasedRandomWalk.cpp:20-28); on a graph the caller declared symmetric,
// x in row(t) when that row is shorter (the same answer there).
__device__ __forceinline__ void n2v_search_rows(int32_t symmetric, int32_t x, int32_t bx,
                                                int32_t dx, int32_t t, int32_t bt, int32_t dt,
                                                int32_t& lo, int32_t& hi, int32_t& tgt) {
    if (symmetric && dt < dx) {
        lo = bt;
        hi = bt + dt;
        tgt = x;
    } else {
        lo = bx;
        hi = bx + dx;
        tgt = t;
    }
}

// Decision once the search has answered whether t is in row(x).  Both
// compares are made and the answer selects between them: selecting the
// threshold instead lets the compiler turn the two argument reads into one
// per-lane load from the kernel-argument segment, a memory round trip (and a
// wait for every store in flight) in the middle of the iteration.
template <int kRule>
__device__ __forceinline__ bool n2v_resolve(const N2VRecArgs& a, float r, bool adjacent) {
    if (kRule == MLXC_RULE_REF_CHAIN) return adjacent;  // only searched when r < p1 decides
    const bool lt1 = r < a.thr1, lt2 = r < a.thr2;
    return adjacent ? lt1 : lt2;
}

// Walks a wavefront of the record walk still holds when the queue has run
// dry and at most this many remain (0: no tail phase): the wavefront then
// finishes them in n2v_tail.  Measured on MI355X at configuration 3 (walk
// kernel): 8.72 ms without the tail phase, 8.68 / 8.62 / 8.55 ms with 8 / 16
// / 32; configuration 5x (about one trial per step) unchanged.
#ifndef MLXC_N2V_TAIL_WALKS
#define MLXC_N2V_TAIL_WALKS 32
#endif
constexpr int kTailWalks = MLXC_N2V_TAIL_WALKS;
static_assert(kTailWalks <= kWave / 2, "a tail walk gets two lanes at least");
constexpr int kTailWords = 13;  // one walk's state in the tail table (below)
static_assert(kTailWalks * kTailWords <= kWave * 8, "the table lives in the wave's staging area");

// Stores, by this lane alone, what a window holds for the output: the block
// and the run deferred to ow_drain, and the entries it buffers, the newest
// of which belongs at last.  (Static indices keep the window in registers.)
template <typename OutT, typename T>
__device__ __forceinline__ void tail_flush(const OutWin<T>& o, OutT* last) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (o.blk != nullptr && i >= 8 - o.blk_n) static_cast<OutT*>(o.blk)[i] = static_cast<OutT>(o.w[i]);
        if (i >= 8 - o.count) last[i - 7] = static_cast<OutT>(o.w[i]);
    }
    for (int32_t j = 0; j < o.run_n; ++j) static_cast<OutT*>(o.run)[j] = static_cast<OutT>(o.run_val);
}

// Whether t is in row(x) (or, on a graph declared symmetric, x in row(t)),
// answered the way the record walk's search phases answer it: a hub bitmap,
// a row hash table, a scan of an unsorted row or a bisection of a sorted
// one, here as a chain of dependent reads of this lane.
__device__ __forceinline__ bool n2v_tail_adjacent(const N2VRecArgs& a, bool sorted, int32_t x,
                                                  int32_t bx, int32_t dx, int32_t sx, int32_t t,
                                                  int32_t bt, int32_t dt, int32_t s_t) {
    int32_t lo, hi, tgt;
    n2v_search_rows(a.symmetric, x, bx, dx, t, bt, dt, lo, hi, tgt);
    const bool one_block = ((lo ^ (hi - 1)) >> 4) == 0;
    if (!one_block && (sx >= 0 || (a.symmetric && s_t >= 0))) {
        const int32_t blk = sx >= 0 ? sx : s_t;
        const int32_t bit = sx >= 0 ? t : x;
        const uint32_t word = a.hub_bits[static_cast<int64_t>(blk) * a.hub_words + (bit >> 5)];
        return ((word >> (bit & 31)) & 1u) != 0;
    }
    const int32_t* col32 = a.index.level[0];
    if (!one_block && a.hash && hi - lo < kHashMaxDegree) {
        const int32_t nb = hash_buckets(hi - lo);
        const int64_t region = hash_region(lo, tgt == t ? x : t);
        int32_t b = hash_bucket(tgt, nb);
        for (int32_t i = 0; i < nb; ++i) {
            const int32_t* bucket = a.hash + static_cast<int64_t>(kSearchBlock) * (region + b);
            bool found = false, open = false;
#pragma unroll
            for (int j = 0; j < kSearchBlock; ++j) {
                found |= bucket[j] == tgt;
                open |= bucket[j] < 0;
            }
            if (found) return true;
            if (open) return false;
            b = b + 1 == nb ? 0 : b + 1;
        }
        return false;
    }
    if (!sorted) {
        for (int32_t i = lo; i < hi; ++i)
            if (col32[i] == tgt) return true;
        return false;
    }
    int32_t count = hi - lo;
    while (count > 0) {  // lower_bound
        const int32_t half = count >> 1;
        if (col32[lo + half] < tgt) {
            lo += half + 1;
            count -= half + 1;
        } else {
            count = half;
        }
    }
    return lo < hi && col32[lo] == tgt;
}

// The end of a record-walk call, for one wavefront: the walks left in its
// table (kTailWords words each: walk id (2 words), steps taken, trial, t and
// its row and hub slot, v and its row and hub slot, and whether the walk
// has not started).  Each walk runs on a group of G lanes, G as large as
// the walks left allow, which try trials trial .. trial + G - 1 of its step
// at once; the step takes the first of them, in trial order, that accepts
// or meets a malformed record, as one lane trying them in turn would have
// stopped there.  The draws are keyed by (walk, step, trial) and the
// neighbour test has one answer whatever reads it, so the walks are the same
// as in the main loop.  When a walk ends the others are regrouped.  Without
// this phase a call's last walks run one lane each while the device is
// nearly idle: the call's tail is the longest of them.
template <int kRule, bool kEdges, bool kCsr, typename OutT>
__device__ void n2v_tail(const N2VRecArgs& a, int32_t* tab, int live, bool sorted,
                         uint32_t& status) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    OutT* const nout = static_cast<OutT*>(a.w.n_out);
    OutT* const eout = static_cast<OutT*>(a.w.e_out);
    const int64_t L = a.w.walk_length;
    const int lane = __lane_id();
    while (live > 0) {  // wave-uniform
        int G = 2;
        while (2 * G * live <= kWave) G *= 2;
        const int w = lane / G, k = lane % G, base = lane & ~(G - 1);
        const uint64_t group_bits = G == kWave ? ~0ull : (1ull << G) - 1;
        const bool act = w < live;
        int64_t n = 0;
        int32_t l = 0, t = 0, bt = 0, dt = 0, s_t = -1, v = 0, bv = 0, dv = 0, sv = -1;
        uint32_t trial = 0;
        bool fresh = false;
        if (act) {
            const int32_t* rec = tab + w * kTailWords;
            n = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(rec[1])) << 32) |
                                     static_cast<uint32_t>(rec[0]));
            l = rec[2];
            trial = static_cast<uint32_t>(rec[3]);
            t = rec[4];
            bt = rec[5];
            dt = rec[6];
            s_t = rec[7];
            v = rec[8];
            bv = rec[9];
            dv = rec[10];
            sv = rec[11];
            fresh = rec[12] != 0;
        }
        wave_sync();
        const int64_t g0 = n * (L + 1), e0 = n * L;
        bool fin = false;
        // the rest of the walk's row stays at v from entry l + 1 on (edges -1)
        auto fill = [&]() {
            for (int64_t j = l + 1 + k; j <= L; j += G) nout[g0 + j] = static_cast<OutT>(v);
            if (kEdges)
                for (int64_t j = l + k; j < L; j += G) eout[e0 + j] = static_cast<OutT>(-1);
            fin = true;
        };
        if (act && fresh) {
            const i32x4 r0 = *reinterpret_cast<const i32x4*>(a.init + n);
            v = r0.x;
            if (k == 0) nout[g0] = static_cast<OutT>(v);
            l = 0;
            trial = 0;
            if (r0.z < 0) {
                status |= r0.z == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW;
                fill();
            } else if (L == 0) {
                fin = true;
            } else if (r0.z == 0) {
                fill();  // absorbing start node
            } else {
                bv = r0.y;
                dv = r0.z;
                sv = kCsr ? -1 : r0.w;
            }
        }
        while (!__any(act && fin)) {  // rounds until a walk ends
            // trial `trial + k` of step l from v: 0 rejected, 1 accepted, else
            // 4 | the status bit of a malformed record
            const uint32_t my = trial + static_cast<uint32_t>(k);
            int32_t e = bv, x = 0, bx = 0, dx = 0, sx = -1;
            uint32_t outcome = 0;
            if (act) {
                float r = 0.0f;
                if (dv != 1) {  // (a forced step takes its only edge)
                    float u0;
                    n2v_uniforms(a.w.walk_base + n, l, my, a.key0, a.key1, u0, r);
                    e = bv + static_cast<int32_t>(pick_index(u0, dv));
                }
                const bool cap = my == MLXC_MAX_TRIALS - 1;  // the cap keeps the last candidate
                if (!kCsr) {
                    const i32x4 rec = *reinterpret_cast<const i32x4*>(a.recs + e);
                    x = rec.x;
                    bx = rec.y;
                    dx = rec.z;
                    sx = rec.w;
                    if (dx < 0) {
                        outcome = 4u | (dx == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW);
                    } else if (l == 0 || dv == 1) {
                        outcome = 1;  // first step, or a forced step (BiasedRandomWalk.cpp:60-66, 76-78)
                    } else {
                        int d = n2v_decide<kRule>(a, r, x, t);
                        if (d < 0)
                            d = n2v_resolve<kRule>(a, r,
                                                   dx > 0 && n2v_tail_adjacent(a, sorted, x, bx, dx, sx,
                                                                               t, bt, dt, s_t))
                                    ? 1
                                    : 0;
                        outcome = d == 1 || cap ? 1u : 0u;
                    }
                } else {
                    // CSR mode: the candidate's id from col32 (-1: a bad col
                    // entry), its row from row32 when the step or the test
                    // needs it, as the main loop reads them
                    x = a.index.level[0][e];
                    const int d = l == 0 || dv == 1 ? 1 : n2v_decide<kRule>(a, r, x, t);
                    if (static_cast<uint32_t>(x) >= static_cast<uint32_t>(a.w.num_nodes)) {
                        outcome = 4u | MLXC_STATUS_BAD_NODE;
                    } else if (d == 0 && !cap) {
                        outcome = 0;
                    } else if (d != -1 && x == t && l > 0) {
                        outcome = 1;  // back to t, whose row the walk keeps
                        bx = bt;
                        dx = dt;
                    } else {
                        typedef int32_t i32x2 __attribute__((ext_vector_type(2), aligned(4)));
                        const i32x2 rr = *reinterpret_cast<const i32x2*>(a.row32 + x);
                        bx = rr.x;
                        dx = rr.y - rr.x;
                        if (rr.x < 0 || rr.y < rr.x) {
                            outcome = 4u | MLXC_STATUS_BAD_ROW;
                        } else if (d != -1) {
                            outcome = 1;
                        } else {
                            const bool acc = n2v_resolve<kRule>(
                                a, r, dx > 0 && n2v_tail_adjacent(a, sorted, x, bx, dx, -1, t, bt, dt, -1));
                            outcome = acc || cap ? 1u : 0u;
                        }
                    }
                }
            }
            const uint64_t decided = (__ballot(outcome != 0) >> base) & group_bits;
            if (!act) continue;
            if (decided == 0) {
                trial += static_cast<uint32_t>(G);
                continue;
            }
            const int src = base + __builtin_ctzll(decided);
            outcome = __shfl(outcome, src, kWave);
            x = __shfl(x, src, kWave);
            e = __shfl(e, src, kWave);
            bx = __shfl(bx, src, kWave);
            dx = __shfl(dx, src, kWave);
            sx = __shfl(sx, src, kWave);
            if (outcome != 1) {
                status |= outcome & 3u;
                fill();
                continue;
            }
            if (k == 0) {
                nout[g0 + l + 1] = static_cast<OutT>(x);
                if (kEdges) eout[e0 + l] = static_cast<OutT>(e);
            }
            l += 1;
            t = v;
            bt = bv;
            dt = dv;
            s_t = sv;
            v = x;
            bv = bx;
            dv = dx;
            sv = sx;
            trial = 0;
            if (l == L) {
                fin = true;
            } else if (dv == 0) {
                fill();
            }
        }
        // the walks that go on, back into the table in order
        const uint64_t keep = __ballot(act && !fin && k == 0);
        if (act && !fin && k == 0) {
            int32_t* rec = tab + lane_rank(keep) * kTailWords;
            rec[0] = static_cast<int32_t>(static_cast<uint32_t>(n));
            rec[1] = static_cast<int32_t>(static_cast<uint32_t>(static_cast<uint64_t>(n) >> 32));
            rec[2] = l;
            rec[3] = static_cast<int32_t>(trial);
            rec[4] = t;
            rec[5] = bt;
            rec[6] = dt;
            rec[7] = s_t;
            rec[8] = v;
            rec[9] = bv;
            rec[10] = dv;
            rec[11] = sv;
            rec[12] = 0;
        }
        wave_sync();
        live = __popcll(keep);
    }
}

// node2vec walk over edge records (num_nodes, num_edges below 2^31; n_out and
// e_out 16-byte aligned).  One walk per lane slot from the wave queue.  Every
// iteration a live slot issues one dependent read: its start record or its
// candidate's edge record (16 bytes; the record carries the candidate's row,
// so the neighbour test needs no rowptr read), or one 64-byte block of the
// neighbour search; the read is unconditional (idle slots read the first
// start record) and the wave waits once.  Sorted rows are searched through
// the index levels (level_step); unsorted rows are scanned 16 entries per
// read, as the reference scans them.  In record mode a wavefront's last
// walks (queue empty, at most kTailWalks left) finish in n2v_tail.
//
// kCsr (CSR mode, for calls with few steps per edge, where building a record
// per edge costs more than it saves): a candidate is read as its col32 entry
// alone, and its row from rowptr only when the decision needs it — to take
// the step, or to search it.  A rejected trial costs one read either way; an
// accepted one two (one when the walk returns to t, whose row it keeps).
template <int kRule, bool kEdges, bool kCsr, typename OutT>
__global__ __launch_bounds__(kBlock) void node2vec_rec_kernel(N2VRecArgs a) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    typedef int32_t i32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    OutT* const nout = static_cast<OutT*>(a.w.n_out);
    OutT* const eout = static_cast<OutT*>(a.w.e_out);
    const bool sorted = a.rows == MLXC_ROWS_SORTED ||
                        (a.rows == MLXC_ROWS_DETECT && a.w.work[2] == a.w.work[3]);
    const int64_t L = a.w.walk_length;
    const int64_t N = a.w.num_walks;
    // the index levels lie after level 0 in one workspace: 32-bit offsets
    // (in entries) select a lane's level more cheaply than 64-bit pointers
    uint32_t level_off[kMaxLevels];
#pragma unroll
    for (int k = 0; k < kMaxLevels; ++k)
        level_off[k] = k < a.index.count ? static_cast<uint32_t>(a.index.level[k] - a.index.level[0]) : 0u;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.w.work + 1);
    WaveQueue q{0, 0};
    int phase = kN2vIdle;
    int64_t n = 0;
    int64_t e0 = 0, g0 = 0; // output index of the walk's edge 0 (n L) and node 0 (n (L + 1))
    int32_t l = 0;          // steps done
    uint32_t trial = 0;
    int32_t t = 0, bt = 0, dt = 0;   // previous node and (CSR mode) its row
    int32_t v = 0, bv = 0, dv = 0;   // current node and its row
    int row_then = kRowAccept;       // CSR mode: what the row read is for
    int32_t e = 0;          // candidate edge
    int32_t x = 0, bx = 0, dx = 0;   // candidate node and its row (from its record)
    int lvl = 0;            // search: index level of the block to read next
    int32_t blk = 0;        // search: that block (kN2vLevel)
    int32_t lo = 0, hi = 0; // search: col32 positions that can still hold tgt
    int32_t tgt = 0;        // search: the node looked for (t in row(x), or x in row(t))
    int32_t sx = -1, sv = -1, s_t = -1;  // hub bitmap slots of x, v and t (-1: none)
    float r = 0.0f;         // acceptance uniform of the current trial
    OutWin<int32_t> ow;
    OutWin<int32_t> ew;     // edge ids (kEdges): e_out[n*L + l] is step l's edge
    ow_init(ow);
    ow_init(ew);
    __shared__ WaveStage stage[kBlock / kWave];
    WaveStage& st = stage[threadIdx.x / kWave];
    uint32_t status = 0;
    if (kTailWalks > 0 && a.tail_direct > 0) {
        // A call of few walks: wavefront k takes walks [k d, k d + d) with
        // d = tail_direct and runs them in n2v_tail from their start, a
        // group of lanes each; no queue.
        const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
        const int64_t w0 = wave * a.tail_direct;
        const int64_t left = N - w0;
        const int cnt = left <= 0 ? 0 : left < a.tail_direct ? static_cast<int>(left) : a.tail_direct;
        int32_t* tab = &st.vals[0][0];
        const int lane = __lane_id();
        if (lane < cnt) {
            int32_t* rec = tab + lane * kTailWords;
            const int64_t id = w0 + lane;
            rec[0] = static_cast<int32_t>(static_cast<uint32_t>(id));
            rec[1] = static_cast<int32_t>(static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32));
            for (int k = 2; k < kTailWords - 1; ++k) rec[k] = 0;
            rec[kTailWords - 1] = 1;  // not started
        }
        wave_sync();
        n2v_tail<kRule, kEdges, kCsr, OutT>(a, tab, cnt, sorted, status);
        if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
        return;
    }
    bool drained = false;  // the queue has run dry (wave-uniform)
    bool tail = false;     // the wavefront's last walks go to n2v_tail

    while (true) {
        // 1. This iteration's read: 16 bytes (a record, the aligned 16 bytes
        // of col32 holding a candidate, or a rowptr pair), or a whole 64-byte
        // block of an index level in the search phases (col32 and every
        // level are padded to whole blocks).
        const int ph = phase;
        const int32_t* bp;
        if (ph == kN2vStart) {
            bp = reinterpret_cast<const int32_t*>(a.init + n);
        } else if (ph == kN2vCand) {
            if (kCsr)
                bp = a.index.level[0] + (e & ~3);  // the aligned 16 bytes holding col32[e]
            else
                bp = reinterpret_cast<const int32_t*>(a.recs + e);
        } else if (kCsr && ph == kN2vRow) {
            bp = a.row32 + x;  // row32[x], row32[x + 1] (4-byte aligned)
        } else if (ph == kN2vLevel) {
            uint32_t off = 0;  // level lvl's offset from level 0, in entries
#pragma unroll
            for (int k = 1; k < kMaxLevels; ++k)
                if (lvl == k) off = level_off[k];
            bp = a.index.level[0] + off + static_cast<int64_t>(kSearchBlock) * blk;
        } else if (ph == kN2vScan) {
            bp = a.index.level[0] + (lo & ~(kSearchBlock - 1));
        } else if (!kCsr && ph == kN2vBit) {
            // the aligned 16 bytes holding word tgt / 32 of bitmap blk
            bp = reinterpret_cast<const int32_t*>(a.hub_bits + blk * a.hub_words +
                                                  ((tgt >> 5) & ~3));
        } else if (!kCsr && ph == kN2vHash) {
            bp = a.hash + static_cast<int64_t>(kSearchBlock) * blk;  // bucket blk
        } else {
            bp = reinterpret_cast<const int32_t*>(a.init);
        }
        i32x4 qb[4];
        if (kCsr)
            qb[0] = *reinterpret_cast<const i32x4a4*>(bp);
        else
            qb[0] = reinterpret_cast<const i32x4*>(bp)[0];
        // the other 48 bytes of the block only for the search phases (reading
        // them for every phase costs registers and measured slower at C5)
        if (ph == kN2vLevel || ph == kN2vScan || (!kCsr && ph == kN2vHash)) {
#pragma unroll
            for (int i = 1; i < 4; ++i) qb[i] = reinterpret_cast<const i32x4*>(bp)[i];
        }
        // ... and the output blocks the last iteration completed are stored.
        ow_drain<OutT>(ow, st);
        if (kEdges) ow_drain<OutT>(ew, st);

        // 2. Idle slots draw walk ids while the read is in flight.
        const bool need = phase == kN2vIdle;
        const int64_t id = queue_take(q, need, counter);
        if (need) {
            n = id;
            l = 0;
            e0 = n * L;
            g0 = e0 + n;
            phase = id < N ? kN2vStart : kN2vDone;
        }
        if (!__any(phase != kN2vDone)) break;
        if (kTailWalks > 0) drained = drained || __any(phase == kN2vDone);
        wait_vmem();
        if (ph != kN2vIdle && ph != kN2vDone) {
            const i32x4 rec = qb[0];

            // 3. Consume.
            bool push = false, fill = false, flush = false, accept = false, next_trial = false;
            bool draw = false;  // draw trial `trial` of step l from v's row (bv, dv)
            int64_t g = g0 + l;  // output index of the last buffered entry
            if (ph == kN2vStart) {
                ow.count = 0;
                ew.count = 0;
                v = rec.x;
                sv = kCsr ? -1 : rec.w;
                push = true;
                if (rec.z < 0) {
                    status |= rec.z == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW;
                    fill = true;
                } else if (L == 0) {
                    flush = true;
                } else if (rec.z == 0) {
                    fill = true;  // absorbing start node
                } else {
                    // first step: uniform, no acceptance test (BiasedRandomWalk.cpp:60-66)
                    bv = rec.y;
                    dv = rec.z;
                    trial = 0;
                    draw = true;
                    phase = kN2vCand;
                }
            } else if (kCsr && ph == kN2vCand) {
                const int k = e & 3;
                x = k == 0 ? rec.x : k == 1 ? rec.y : k == 2 ? rec.z : rec.w;
                int d = 1;  // first step and forced steps accept
                if (!(l == 0 || dv == 1)) d = n2v_decide<kRule>(a, r, x, t);
                if (static_cast<uint32_t>(x) >= static_cast<uint32_t>(a.w.num_nodes)) {
                    status |= MLXC_STATUS_BAD_NODE;  // (col32 holds -1 for any bad col)
                    fill = true;
                } else if (d == 0) {
                    next_trial = true;
                } else if (d == 1 && x == t && l > 0) {
                    accept = true;  // back to t: its row is known
                    bx = bt;
                    dx = dt;
                } else {
                    row_then = d == 1 ? kRowAccept : kRowSearch;
                    phase = kN2vRow;
                }
            } else if (kCsr && ph == kN2vRow) {
                // row32[x] and row32[x + 1] (-1 marks an entry outside [0, num_edges])
                const bool ok = rec.x >= 0 && rec.y >= rec.x;
                bx = rec.x;
                dx = rec.y - rec.x;
                if (!ok) {
                    status |= MLXC_STATUS_BAD_ROW;
                    fill = true;
                } else if (row_then == kRowAccept) {
                    accept = true;
                } else if (dx == 0) {
                    accept = n2v_resolve<kRule>(a, r, false);
                    next_trial = !accept;
                } else {
                    n2v_search_rows(a.symmetric, x, bx, dx, t, bt, dt, lo, hi, tgt);
                    if (!sorted) {
                        phase = kN2vScan;
                    } else {
                        const uint32_t diff = static_cast<uint32_t>(lo) ^ static_cast<uint32_t>(hi - 1);
                        lvl = diff ? (31 - __builtin_clz(diff)) >> 2 : 0;
                        blk = static_cast<int32_t>(static_cast<int64_t>(lo) >> (4 * (lvl + 1)));
                        phase = kN2vLevel;
                    }
                }
            } else if (ph == kN2vCand) {
                x = rec.x;
                bx = rec.y;
                dx = rec.z;
                sx = rec.w;
                if (dx < 0) {
                    status |= dx == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW;
                    fill = true;
                } else if (l == 0 || dv == 1) {
                    accept = true;  // first step, or a forced step (BiasedRandomWalk.cpp:76-78)
                } else {
                    const int d = n2v_decide<kRule>(a, r, x, t);
                    if (d == 1) {
                        accept = true;
                    } else if (d == 0) {
                        next_trial = true;
                    } else if (dx == 0) {
                        accept = n2v_resolve<kRule>(a, r, false);
                        next_trial = !accept;
                    } else {
                        n2v_search_rows(a.symmetric, x, bx, dx, t, bt, dt, lo, hi, tgt);
                        // a row inside one aligned 16-entry block takes one read
                        // either way; longer ones take the bitmap's single read
                        const bool one_block = ((lo ^ (hi - 1)) >> 4) == 0;
                        if (!one_block && sx >= 0) {
                            blk = sx;  // bit t of row(x)'s bitmap
                            tgt = t;
                            phase = kN2vBit;
                        } else if (!one_block && a.symmetric && s_t >= 0) {
                            blk = s_t;  // bit x of row(t)'s bitmap: the same answer on a symmetric graph
                            tgt = x;
                            phase = kN2vBit;
                        } else if (!one_block && a.hash && hi - lo < kHashMaxDegree) {
                            // the row searched has no bitmap (it would have been
                            // taken above) and a hash table: lo <- its first
                            // bucket, hi <- its bucket count, blk <- tgt's bucket
                            const int32_t node = tgt == t ? x : t;
                            const int32_t nb = hash_buckets(hi - lo);
                            lo = static_cast<int32_t>(hash_region(lo, node));
                            hi = nb;
                            blk = lo + hash_bucket(tgt, nb);
                            lvl = 0;  // buckets read
                            phase = kN2vHash;
                        } else if (!sorted) {
                            phase = kN2vScan;
                        } else {
                            // finest level whose aligned blocks (16^(lvl+1) positions)
                            // hold the whole row in one
                            const uint32_t diff = static_cast<uint32_t>(lo) ^ static_cast<uint32_t>(hi - 1);
                            lvl = diff ? (31 - __builtin_clz(diff)) >> 2 : 0;
                            blk = static_cast<int32_t>(static_cast<int64_t>(lo) >> (4 * (lvl + 1)));
                            phase = kN2vLevel;
                        }
                    }
                }
            } else if (!kCsr && ph == kN2vBit) {
                const uint32_t word = static_cast<uint32_t>(rec[(tgt >> 5) & 3]);
                accept = n2v_resolve<kRule>(a, r, ((word >> (tgt & 31)) & 1u) != 0);
                next_trial = !accept;
            } else if (!kCsr && ph == kN2vHash) {
                // tgt in the bucket: adjacent; an empty slot (-1): not adjacent;
                // a full bucket without tgt: the next bucket of the table.  A
                // table always has an empty slot; the bound on the buckets read
                // only keeps a malformed CSR (rows that overlap, whose tables
                // then overwrite each other) from looping.
                bool found = false, open = false;
    #pragma unroll
                for (int i = 0; i < kSearchBlock; ++i) {
                    const int32_t v16 = qb[i / 4][i % 4];
                    found |= v16 == tgt;
                    open |= v16 < 0;
                }
                lvl += 1;
                if (found || open || lvl >= hi) {
                    accept = n2v_resolve<kRule>(a, r, found);
                    next_trial = !accept;
                } else {
                    blk = blk + 1 == lo + hi ? lo : blk + 1;
                }
            } else {  // the neighbour search: is t in row(x)?
                int32_t vals[kSearchBlock];
    #pragma unroll
                for (int i = 0; i < kSearchBlock; ++i) vals[i] = qb[i / 4][i % 4];
                const int res = ph == kN2vLevel ? level_step(vals, tgt, lvl, blk, lo, hi)
                                                : scan_step(vals, tgt, lo, hi);
                if (res >= 0) {
                    accept = n2v_resolve<kRule>(a, r, res == 1);
                    next_trial = !accept;
                }
            }
            if (next_trial) {
                trial += 1;
                if (trial >= MLXC_MAX_TRIALS) {
                    // trial cap: keep the last candidate (CSR mode: read its row
                    // first, unless it is t)
                    if (!kCsr) {
                        accept = true;
                    } else if (x == t) {
                        accept = true;
                        bx = bt;
                        dx = dt;
                    } else {
                        row_then = kRowAccept;
                        phase = kN2vRow;
                    }
                } else {
                    draw = true;
                    phase = kN2vCand;
                }
            }
            if (accept) {
                if (kEdges) ow_push(ew, eout, e0 + l, e);
                push = true;
                g += 1;
                l += 1;
                t = v;
                bt = bv;
                dt = dv;
                s_t = sv;
                v = x;
                bv = bx;
                dv = dx;
                sv = sx;
                if (l == L) {
                    flush = true;
                } else if (dv == 0) {
                    fill = true;
                } else {
                    trial = 0;
                    if (dv == 1)
                        e = bv;  // forced: no draw
                    else
                        draw = true;
                    phase = kN2vCand;
                }
            }
            // The trial's candidate and r: one Philox call site for the three
            // places that draw (a wavefront executes each site any lane needs).
            if (draw) {
                float u0;
                n2v_uniforms(a.w.walk_base + n, l, trial, a.key0, a.key1, u0, r);
                e = bv + static_cast<int32_t>(pick_index(u0, dv));
            }
            if (fill) {
                ow_fill(ow, nout, push ? g : g + 1, g0 + L, v);  // v from g on
                if (kEdges) ow_fill(ew, eout, e0 + l, e0 + L - 1, -1);  // l edges buffered
            } else {
                if (push) ow_push(ow, nout, g, v);
                if (flush) {
                    if (ow.count) ow_flush(ow, nout, g);
                    if (kEdges && ew.count) ow_flush(ew, eout, e0 + L - 1);
                }
            }
            if (fill || flush) phase = kN2vIdle;
        }
        // 4. Once the queue has run dry and at most kTailWalks walks are left
        // to the wavefront (a lane whose walk just ended takes no other),
        // n2v_tail finishes them.  (Checked here, where every lane has
        // reconverged and no read is in flight: the register allocation of
        // the loop then stays as it is without the tail.)
        if (kTailWalks > 0 && drained &&
            __popcll(__ballot(phase != kN2vDone && phase != kN2vIdle)) <= kTailWalks) {
            tail = true;
            break;
        }
    }
    if (tail) {
        // The stores this iteration deferred, and the entries the windows
        // still hold (the walk's newest at g0 + l, its edges' at e0 + l - 1),
        // stored here by each lane for itself.  A trial in progress is tried
        // again from its draw in n2v_tail.
        tail_flush<OutT>(ow, nout + g0 + l);
        if (kEdges) tail_flush<OutT>(ew, eout + e0 + l - 1);
        const bool live = phase != kN2vDone && phase != kN2vIdle;
        const uint64_t mask = __ballot(live);
        int32_t* tab = &st.vals[0][0];
        wave_sync();
        if (live) {
            int32_t* rec = tab + lane_rank(mask) * kTailWords;
            rec[0] = static_cast<int32_t>(static_cast<uint32_t>(n));
            rec[1] = static_cast<int32_t>(static_cast<uint32_t>(static_cast<uint64_t>(n) >> 32));
            rec[2] = l;
            rec[3] = static_cast<int32_t>(trial);
            rec[4] = t;
            rec[5] = bt;
            rec[6] = dt;
            rec[7] = s_t;
            rec[8] = v;
            rec[9] = bv;
            rec[10] = dv;
            rec[11] = sv;
            rec[12] = phase == kN2vStart;
        }
        wave_sync();
        n2v_tail<kRule, kEdges, kCsr, OutT>(a, tab, __popcll(mask), sorted, status);
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// node2vec walk on a graph small enough for LDS (lds_walk_fits), for calls
// bound by launch latency (the reference tests' Cora-sized workload): every
// block copies rowptr and col, as int32, into its LDS; each walk runs on a
// group of lds_group consecutive lanes, with the same draws and decisions as
// the record walk, the neighbour test by bisection (sorted rows) or a linear
// scan (unsorted rows) in LDS.  Every
// block validates its copy of the whole CSR, as the preparation passes of the
// other layouts do (block 0 reports it); with MLXC_ROWS_DETECT each block
// also decides the row order of its copy by the preparation passes' rule
// (CsrCheck: every position i >= 1 with col[i] < col[i-1] starts a non-empty
// row), checked entry-parallel.
template <int kRule, bool kEdges, typename OutT>
__global__ __launch_bounds__(kLdsBlock) void node2vec_lds_kernel(N2VRecArgs a) {
    __shared__ int32_t graph[kLdsGraphEntries];
    const int64_t V = a.w.num_nodes, E = a.w.num_edges, N = a.w.num_walks, L = a.w.walk_length;
    int32_t* const rp = graph;          // rowptr, -1 for an entry outside [0, E]
    int32_t* const cl = graph + V + 1;  // col, -1 for a value outside [0, V)
    bool bad_row = false, bad_col = false;
    for (int64_t i = threadIdx.x; i <= V; i += kLdsBlock) {
        const int64_t r = a.w.rowptr[i];
        const bool ok = r >= 0 && r <= E;
        rp[i] = ok ? static_cast<int32_t>(r) : -1;
        bad_row |= !ok || (i == 0 && r != 0) || (i == V && r != E);
    }
    for (int64_t i = threadIdx.x; i < E; i += kLdsBlock) {
        const int64_t c = a.w.col[i];
        const bool ok = node_ok(c, V);
        cl[i] = ok ? static_cast<int32_t>(c) : -1;
        bad_col |= !ok;
    }
    __syncthreads();
    for (int64_t u = threadIdx.x; u < V; u += kLdsBlock) bad_row |= rp[u + 1] < rp[u];
    // (every reduction below is a block-wide barrier every thread reaches)
    const bool any_bad_row = __syncthreads_or(bad_row);
    const bool any_bad_col = __syncthreads_or(bad_col);
    bool sorted = a.rows == MLXC_ROWS_SORTED;
    if (a.rows == MLXC_ROWS_DETECT) {
        // the block's descents minus those at a row start (each of which is
        // also a descent): zero exactly when the rows are sorted
        __shared__ int extra;
        if (threadIdx.x == 0) extra = 0;
        __syncthreads();
        int d = 0;
        for (int64_t i = 1 + threadIdx.x; i < E; i += kLdsBlock) d += cl[i] < cl[i - 1];
        for (int64_t u = threadIdx.x; u < V; u += kLdsBlock) {
            const int32_t b = rp[u], end = rp[u + 1];
            d -= b >= 1 && end > b && cl[b] < cl[b - 1];
        }
        // one LDS atomic per wavefront (one per thread serialized on the
        // word: 3.4 us of the reference test's 31 us call)
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) d += __shfl_xor(d, off, kWave);
        if (__lane_id() == 0 && d) atomicAdd(&extra, d);
        __syncthreads();
        sorted = extra == 0;
    }
    OutT* const nout = static_cast<OutT*>(a.w.n_out);
    OutT* const eout = static_cast<OutT*>(a.w.e_out);
    uint32_t status = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        status = (any_bad_row ? MLXC_STATUS_BAD_ROW : 0u) | (any_bad_col ? MLXC_STATUS_BAD_NODE : 0u);
    // One round of trials per loop iteration: the G = lds_group lanes of a
    // walk try trials trial .. trial + G - 1 of its step at once, one each,
    // and the step takes the first of them, in trial order, that accepts (or
    // meets a malformed entry), which is where one lane trying them in turn
    // would have stopped: the same walks, in fewer rounds.  A call with few
    // walks leaves most of the device idle, and its time is the longest
    // chain of trials of one walk; G lanes cut that chain about G-fold where
    // steps take several trials.  A walk that takes its step goes on with
    // the next step (or its next walk) in the next iteration, so a wavefront
    // runs as long as its longest walk.  Every lane of a group holds the
    // walk's whole state; only the trial differs.
    const int G = a.lds_group;
    const int k = static_cast<int>(threadIdx.x) & (G - 1);  // this lane's trial offset
    const int base = __lane_id() & ~(G - 1);                 // the group's first lane
    const uint32_t group_bits = (G == 32 ? 0xffffffffu : (1u << G) - 1u);
    const int64_t walkers = a.lds_walkers;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * walkers;
    const int64_t gi = threadIdx.x / G;
    int64_t n = gi < walkers ? static_cast<int64_t>(blockIdx.x) * walkers + gi : N;
    OutT* row = nullptr;
    OutT* erow = nullptr;
    int64_t l = 0;           // steps taken
    int32_t v = 0, t = 0;    // current and previous node
    int32_t b = 0, deg = 0;  // row of v
    uint32_t trial = 0;
    bool walking = false;    // walk n has a trial due
    // the walk stays at v from step l on (the group's lanes share the
    // stores); then the group takes its next walk
    auto finish = [&]() {
        for (int64_t j = l + 1 + k; j <= L; j += G) row[j] = static_cast<OutT>(v);
        if (kEdges)
            for (int64_t j = l + k; j < L; j += G) erow[j] = static_cast<OutT>(-1);
        walking = false;
        n += stride;
    };
    while (true) {
        if (!walking) {
            if (n >= N) break;
            const int64_t s = a.w.start[n];
            row = nout + n * (L + 1);
            erow = kEdges ? eout + n * L : nullptr;
            if (k == 0) row[0] = static_cast<OutT>(s);
            l = 0;
            v = static_cast<int32_t>(s);
            t = v;
            if (!node_ok(s, V)) {
                status |= MLXC_STATUS_BAD_NODE;
                finish();
                continue;
            }
            if (L == 0) {
                finish();
                continue;
            }
            b = rp[v];
            const int32_t end = rp[v + 1];
            if (b < 0 || end < b) {
                status |= MLXC_STATUS_BAD_ROW;
                finish();
                continue;
            }
            deg = end - b;
            if (deg == 0) {  // absorbing start node: the walk stays
                finish();
                continue;
            }
            trial = 0;
            walking = true;
        }
        // trial `trial + k` of step l from v; the first step and forced steps
        // accept at trial 0 (BiasedRandomWalk.cpp:60-66, 76-78), and the
        // trial cap keeps the last candidate
        const uint32_t my = trial + static_cast<uint32_t>(k);
        const bool test = l > 0 && deg > 1;
        float r = 0.0f;
        int32_t e = b;
        if (l == 0 || deg > 1) {
            float u0;
            n2v_uniforms(a.w.walk_base + n, static_cast<int32_t>(l), my, a.key0, a.key1, u0, r);
            e = b + static_cast<int32_t>(pick_index(u0, deg));
        }
        int32_t x = cl[e];
        int32_t bx = x >= 0 ? rp[x] : -1, ex = x >= 0 ? rp[x + 1] : -1;
        // 0: rejected, 1: accepted, else the status bit of a malformed entry
        uint32_t outcome = 1;
        if (x < 0) {
            outcome = MLXC_STATUS_BAD_NODE | 4u;
        } else if (bx < 0 || ex < bx) {
            outcome = MLXC_STATUS_BAD_ROW | 4u;
        } else if (test) {
            int d = n2v_decide<kRule>(a, r, x, t);
            if (d < 0) {  // is t in row(x)?
                bool adjacent = false;
                if (sorted) {
                    int32_t lo = bx, count = ex - bx;
                    while (count > 0) {  // lower_bound
                        const int32_t half = count >> 1;
                        if (cl[lo + half] < t) {
                            lo += half + 1;
                            count -= half + 1;
                        } else {
                            count = half;
                        }
                    }
                    adjacent = lo < ex && cl[lo] == t;
                } else {
                    for (int32_t i = bx; i < ex && !adjacent; ++i) adjacent = cl[i] == t;
                }
                d = n2v_resolve<kRule>(a, r, adjacent) ? 1 : 0;
            }
            outcome = d == 1 || my == MLXC_MAX_TRIALS - 1 ? 1u : 0u;
        }
        // the group's first trial that does not reject (the group's lanes
        // reach this point together: their control flow up to here depends
        // on the walk's state alone, apart from the search above)
        const uint32_t decided =
            static_cast<uint32_t>(__ballot(outcome != 0) >> base) & group_bits;
        if (decided == 0) {
            trial += static_cast<uint32_t>(G);
            continue;
        }
        const int src = base + __builtin_ctz(decided);
        outcome = __shfl(outcome, src, kWave);
        x = __shfl(x, src, kWave);
        e = __shfl(e, src, kWave);
        bx = __shfl(bx, src, kWave);
        ex = __shfl(ex, src, kWave);
        if (outcome != 1) {
            status |= outcome & 3u;
            finish();
            continue;
        }
        // the step to x, whose row the trial has read and checked
        if (k == 0) {
            row[l + 1] = static_cast<OutT>(x);
            if (kEdges) erow[l] = static_cast<OutT>(e);
        }
        t = v;
        v = x;
        l += 1;
        b = bx;
        deg = ex - bx;
        trial = 0;
        if (l == L || deg == 0) finish();  // (deg 0: an absorbing node, the walk stays)
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------------------------- launcher

namespace {

template <int kRule, bool kEdges, typename OutT>
int launch_n2v(const N2VArgs& a, hipStream_t stream) {
    auto kernel = node2vec_walk_kernel<kRule, kEdges, OutT>;
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid)) return rc;
    if (int rc = record_walk_event(0, stream)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return record_walk_event(1, stream);
}

template <int kRule, typename OutT>
int dispatch_n2v(const N2VArgs& a, bool edges, hipStream_t stream) {
    return edges ? launch_n2v<kRule, true, OutT>(a, stream) : launch_n2v<kRule, false, OutT>(a, stream);
}

// Resident blocks per compute unit of the node2vec record walk (0: as many
// as its registers allow, 5), per rule: the two rules are different kernels.
// Measured on MI355X with 4 blocks and at the limit: the reference chain at
// configuration 3 11.95 and 12.15 ms, with the symmetric hint 11.33 and
// 11.51, configuration 5 (CSR mode) 8.55 and 8.57; the analytic rule at
// configuration 5x 18.25 and 17.55 ms, with the symmetric hint 17.31 and
// 16.61.  The reference-chain walk at configuration 3 spends more of each
// iteration in VALU work (more waves then contend), the analytic walk at 5x
// more of it waiting on reads (more waves hide them).
// Most lanes one walk of the node2vec LDS walk runs on (a power of two, at
// most 32): each tries one trial of the walk's step per round.
#ifndef MLXC_LDS_MAX_GROUP
#define MLXC_LDS_MAX_GROUP 16
#endif

#ifndef MLXC_N2V_BLOCKS_PER_CU
#define MLXC_N2V_BLOCKS_PER_CU 4
#endif
#ifndef MLXC_N2V_ANALYTIC_BLOCKS_PER_CU
#define MLXC_N2V_ANALYTIC_BLOCKS_PER_CU 0
#endif

template <int kRule, bool kEdges, bool kCsr, typename OutT>
int launch_n2v_rec(const N2VRecArgs& a, hipStream_t stream) {
    auto kernel = node2vec_rec_kernel<kRule, kEdges, kCsr, OutT>;
    constexpr int per_cu = kRule == MLXC_RULE_REF_CHAIN ? MLXC_N2V_BLOCKS_PER_CU
                                                         : MLXC_N2V_ANALYTIC_BLOCKS_PER_CU;
    int grid = 0;
    N2VRecArgs b = a;
    b.tail_direct = 0;
    // A call whose walks fill at most half the device's wavefront slots at
    // one per SIMD (256 lanes a CU) leaves lanes to spare: each walk then gets
    // a group of G lanes (the largest power of two, at most 32, that keeps
    // the call within those slots) in the tail phase, 64 / G walks to a
    // wavefront, from the start.
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    const int64_t N = a.w.num_walks, slots = static_cast<int64_t>(info.cus) * 256;
    if (kTailWalks > 0 && N > 0 && 2 * N <= slots) {
        int G = 2;
        while (G < 32 && 2 * G * N <= slots) G *= 2;
        b.tail_direct = kWave / G;
        const int64_t waves = (N + b.tail_direct - 1) / b.tail_direct;
        grid = static_cast<int>((waves + kBlock / kWave - 1) / (kBlock / kWave));
    } else if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid, per_cu)) {
        return rc;
    }
    if (int rc = record_walk_event(0, stream)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, b);
    MLXC_HIP_TRY(hipGetLastError());
    return record_walk_event(1, stream);
}

// Workspace of the record walk: edge records (record mode only), start
// records, then (128-byte aligned) the levels of the search index — col as
// int32, then its samples every 16^k entries — each padded to whole blocks of
// kSearchBlock entries, then 64 bytes of slack for the block reads of the
// last start records.  Record mode then adds, in this order, the row hash
// tables (num_edges / 8 + num_nodes + 2 buckets of 64 bytes; see row_hashed)
// and the hub bitmaps: the info words, slot_of [V], node_of [max] and the
// bitmaps [max][words], up to kHubBudgetBytes of bitmaps and at most one slot
// per kHubMinDegree entries.  A workspace that ends before the bitmaps runs
// without them, one that ends before the tables without both.
struct N2VLayout {
    size_t level[kMaxLevels];
    int count;
    size_t row32;          // the int32 row starts (row32_kernel), num_nodes + 3 entries
    size_t total_base;     // records (or CSR mode), start records, index, row32
    size_t hash;           // the row hash tables (record mode)
    size_t hash_count, hash_list;  // the tables' build: long rows, counted and listed
    size_t total_no_hubs;  // the layout without hub bitmaps (with the tables)
    size_t hub_info, hub_slot_of, hub_node_of, hub_bits;
    int32_t hub_max;
    int64_t hub_words;
    size_t total;
};

// Bytes of hub bitmaps a record layout reserves at most (0: no bitmaps).
#ifndef MLXC_HUB_BUDGET_BYTES
#define MLXC_HUB_BUDGET_BYTES (int64_t{1} << 30)
#endif
constexpr int64_t kHubBudgetBytes = MLXC_HUB_BUDGET_BYTES;

size_t align128(size_t x) { return (x + 127) & ~static_cast<size_t>(127); }

N2VLayout n2v_layout(int64_t num_nodes, int64_t num_edges, int64_t num_walks, bool records) {
    N2VLayout lay;
    lay.count = index_levels(num_edges);
    size_t pos = kRecordOffset +
                 static_cast<size_t>((records ? num_edges : 0) + num_walks) * sizeof(EdgeRecord);
    pos = align128(pos);
    int64_t entries = num_edges;  // level k has ceil(num_edges / 16^k) entries
    for (int k = 0; k < lay.count; ++k) {
        lay.level[k] = pos;
        const int64_t blocks = (entries + kSearchBlock - 1) / kSearchBlock;
        pos += static_cast<size_t>(blocks) * kSearchBlock * sizeof(int32_t);
        entries = blocks;
    }
    pos += 64;
    // the int32 row starts, two entries of slack for the CSR walk's 16-byte reads
    lay.row32 = align128(pos);
    pos = lay.row32 + static_cast<size_t>(num_nodes + 3) * sizeof(int32_t);
    lay.total_base = pos;
    lay.hash = lay.hash_list = lay.hash_count = 0;
    if (records) {
        lay.hash = align128(pos);
        pos = lay.hash + static_cast<size_t>(num_edges / 8 + num_nodes + 2) * kSearchBlock *
                             sizeof(int32_t);
        lay.hash_count = align128(pos);  // the build's count of long rows, then its list
        lay.hash_list = lay.hash_count + 128;
        pos = lay.hash_list + static_cast<size_t>(num_nodes) * sizeof(int32_t);
    }
    lay.total_no_hubs = pos;
    lay.hub_words = ((num_nodes + 31) / 32 + 3) / 4 * 4;
    const int64_t bitmap_bytes = lay.hub_words * 4;
    int64_t max = records && num_nodes > 0 && kHubBudgetBytes > 0 ? num_edges / kHubMinDegree : 0;
    if (bitmap_bytes > 0 && max > kHubBudgetBytes / bitmap_bytes) max = kHubBudgetBytes / bitmap_bytes;
    lay.hub_max = static_cast<int32_t>(max);
    lay.total = lay.total_no_hubs;
    lay.hub_info = lay.hub_slot_of = lay.hub_node_of = lay.hub_bits = 0;
    if (lay.hub_max > 0) {
        lay.hub_info = align128(lay.total_no_hubs);
        lay.hub_slot_of = align128(lay.hub_info + kHubInfoWords * sizeof(int64_t));
        lay.hub_node_of = align128(lay.hub_slot_of + static_cast<size_t>(num_nodes) * sizeof(int32_t));
        lay.hub_bits = align128(lay.hub_node_of + static_cast<size_t>(max) * sizeof(int32_t));
        lay.total = lay.hub_bits + static_cast<size_t>(max) * static_cast<size_t>(bitmap_bytes);
    }
    return lay;
}

// Edge records cost one random rowptr read and 16 bytes per edge and save a
// rowptr read on every step taken and every row searched; CSR mode wins when
// the call takes few steps per edge and seldom searches.  With w the share
// of draws that can need a search, records pay off when
// steps * (1 + 4 w) >= 4 * edges.  Measured on MI355X: configuration 5
// (1.07 steps per edge, w = 0) 9.0 ms in CSR mode against 11.0 with
// records; configuration 5x (w = 0.75) 21.0 against 19.5; configuration 3
// (5.3 steps per edge) 13.6 either way.
bool n2v_records_pay_off(int64_t num_edges, int64_t num_walks, int32_t walk_length,
                         double search_width) {
    const double steps = static_cast<double>(num_walks) * static_cast<double>(walk_length);
    return steps * (1.0 + 4.0 * search_width) >= 4.0 * static_cast<double>(num_edges) ||
           num_edges <= kSmallGraphEdgesPerStep * walk_length;  // small graphs, as for the uniform walk
}

}  // namespace

double n2v_search_width(const N2VParams& p) {
    if (p.rule == MLXC_RULE_REF_CHAIN) return p.prob1 > p.prob2 ? p.prob1 - p.prob2 : 0.0;
    return p.prob1 > p.prob2 ? p.prob1 - p.prob2 : p.prob2 - p.prob1;
}

size_t node2vec_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                                int32_t walk_length, double search_width) {
    if (num_nodes < 0 || num_edges < 0 || num_walks < 0 || walk_length < 0 ||
        !records_fit(num_nodes, num_edges))
        return MLXC_WORK_WORDS * sizeof(int64_t);
    if (lds_walk_fits(num_nodes, num_edges, num_walks, walk_length))
        return kRecordOffset;  // the LDS walk: its size selects it
    const bool records = n2v_records_pay_off(num_edges, num_walks, walk_length, search_width);
    const N2VLayout lay = n2v_layout(num_nodes, num_edges, num_walks, records);
    // the hash tables and hub bitmaps serve only row searches: none without
    return search_width > 0.0 ? lay.total : lay.total_base;
}

size_t node2vec_layout_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                             int32_t walk_length, int32_t layout) {
    if (num_nodes < 0 || num_edges < 0 || num_walks < 0 || walk_length < 0) return 0;
    switch (layout) {
    case MLXC_N2V_LAYOUT_DIRECT:
        return MLXC_WORK_WORDS * sizeof(int64_t);
    case MLXC_N2V_LAYOUT_LDS:
        return lds_walk_fits(num_nodes, num_edges, num_walks, walk_length) ? kRecordOffset : 0;
    default:
        break;
    }
    if (!records_fit(num_nodes, num_edges)) return 0;
    if (layout == MLXC_N2V_LAYOUT_CSR)
        return n2v_layout(num_nodes, num_edges, num_walks, false).total_base;
    const N2VLayout lay = n2v_layout(num_nodes, num_edges, num_walks, true);
    if (layout == MLXC_N2V_LAYOUT_RECORDS) return lay.total_base;
    if (layout == MLXC_N2V_LAYOUT_RECORDS_HASH) return lay.total_no_hubs;
    if (layout == MLXC_N2V_LAYOUT_RECORDS_FULL) return lay.total;
    return 0;
}

namespace {

// Smallest row degree worth a hub bitmap in this call.  A bitmap costs
// num_nodes / 8 bytes of streamed writes per call and saves about two
// dependent reads on each of the call's searches of its row, about
// deg * rho of them (rho: searches per CSR entry, at least steps * w / E for
// a search share w of the draws).  Counting a dependent read as 4 streamed
// lines of 128 bytes, the bitmap pays off from deg ~ num_nodes / (4096 rho).
// INT64_MAX: the call makes no searches, so no bitmaps.
int64_t n2v_hub_min_degree(const WalkArgs& w, const N2VParams& p) {
    const double width = n2v_search_width(p);
    const double rho = static_cast<double>(w.num_walks) * w.walk_length * width /
                       static_cast<double>(w.num_edges > 0 ? w.num_edges : 1);
    if (!(rho > 0.0)) return INT64_MAX;
    const double d = static_cast<double>(w.num_nodes) / (4096.0 * rho);
    if (d >= 1e18) return INT64_MAX;
    return d > static_cast<double>(kHubMinDegree) ? static_cast<int64_t>(std::ceil(d))
                                                  : kHubMinDegree;
}

template <typename OutT>
int launch_node2vec_typed(const WalkArgs& w, const N2VParams& p, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    const bool aligned = reinterpret_cast<uintptr_t>(w.n_out) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(w.e_out) % 16 == 0;  // e_out may be null
    const N2VLayout lay_rec = n2v_layout(w.num_nodes, w.num_edges, w.num_walks, true);
    const N2VLayout lay_csr = n2v_layout(w.num_nodes, w.num_edges, w.num_walks, false);
    // Records whenever the workspace holds them: node2vec_workspace_bytes
    // asks for them only when they pay off; the row hash tables and the hub
    // bitmaps too when it holds them.  Both serve only the row searches,
    // which a call of search width 0 never makes.
    const bool records = workspace_bytes >= lay_rec.total_base;
    const int64_t hub_min_degree = n2v_hub_min_degree(w, p);
    const bool searches = hub_min_degree < INT64_MAX;
    const bool hash_tables = records && searches && workspace_bytes >= lay_rec.total_no_hubs;
    const bool hub_bitmaps = hash_tables && lay_rec.hub_max > 0 && workspace_bytes >= lay_rec.total;
    if (aligned && records_fit(w.num_nodes, w.num_edges) &&
        (records || workspace_bytes >= lay_csr.total)) {
        const N2VLayout& lay = records ? lay_rec : lay_csr;
        N2VRecArgs a;
        a.w = w;
        char* base = static_cast<char*>(workspace);
        HubBitmaps hubs{};
        if (hub_bitmaps) {
            hubs.slot_of = reinterpret_cast<int32_t*>(base + lay.hub_slot_of);
            hubs.node_of = reinterpret_cast<int32_t*>(base + lay.hub_node_of);
            hubs.bits = reinterpret_cast<uint32_t*>(base + lay.hub_bits);
            hubs.info = reinterpret_cast<int64_t*>(base + lay.hub_info);
            hubs.words = lay.hub_words;
            hubs.max = lay.hub_max;
            if (int rc = launch_hub_bitmaps(w.rowptr, w.col, w.num_nodes, w.num_edges, hubs,
                                            hub_min_degree, stream))
                return rc;
        }
        a.hub_bits = hub_bitmaps ? hubs.bits : nullptr;
        a.hub_words = hubs.words;
        EdgeRecord* recs = records ? reinterpret_cast<EdgeRecord*>(base + kRecordOffset) : nullptr;
        EdgeRecord* init = reinterpret_cast<EdgeRecord*>(base + kRecordOffset) +
                           (records ? w.num_edges : 0);
        IndexLevels index{};
        index.count = lay.count;
        for (int k = 0; k < lay.count; ++k)
            index.level[k] = reinterpret_cast<int32_t*>(base + lay.level[k]);
        // one pass builds the search index and the start records, validates
        // the whole CSR and counts the row descents (MLXC_ROWS_DETECT: the walk
        // reads the result on the device, no host sync)
        int64_t* check = w.work;
        const StartRecords starts{w.start, w.num_walks, init};
        int32_t* row32 = reinterpret_cast<int32_t*>(base + lay.row32);
        if (int rc = records ? launch_edge_records(w.rowptr, w.col, w.num_nodes, w.num_edges, recs,
                                                   index, starts, check, stream, hubs, row32)
                             : launch_edge_index(w.rowptr, w.col, w.num_nodes, w.num_edges, index,
                                                 starts, check, stream, row32))
            return rc;
        a.row32 = row32;
        if (hub_bitmaps)
            if (int rc = launch_hub_build(w.rowptr, w.col, w.num_nodes, hubs, p.rows, w.work, stream))
                return rc;
        a.hash = nullptr;
        if (hash_tables) {
            int32_t* table = reinterpret_cast<int32_t*>(base + lay.hash);
            if (int rc = launch_hash_build(row32, index.level[0], w.num_nodes,
                                           hub_bitmaps ? hubs.info : nullptr, table,
                                           reinterpret_cast<int32_t*>(base + lay.hash_list),
                                           reinterpret_cast<int64_t*>(base + lay.hash_count),
                                           stream))
                return rc;
            a.hash = table;
        }
        a.recs = recs;
        a.init = init;
        a.index = index;
        a.thr0 = float_at_or_above(p.prob0);
        a.thr1 = float_at_or_above(p.prob1);
        a.thr2 = float_at_or_above(p.prob2);
        a.key0 = p.key0;
        a.key1 = p.key1;
        a.rows = p.rows;
        a.symmetric = p.symmetric;
        const bool edges = w.e_out != nullptr;
        if (records) {
            if (p.rule == MLXC_RULE_REF_CHAIN)
                return edges ? launch_n2v_rec<MLXC_RULE_REF_CHAIN, true, false, OutT>(a, stream)
                             : launch_n2v_rec<MLXC_RULE_REF_CHAIN, false, false, OutT>(a, stream);
            return edges ? launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, true, false, OutT>(a, stream)
                         : launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, false, false, OutT>(a, stream);
        }
        if (p.rule == MLXC_RULE_REF_CHAIN)
            return edges ? launch_n2v_rec<MLXC_RULE_REF_CHAIN, true, true, OutT>(a, stream)
                         : launch_n2v_rec<MLXC_RULE_REF_CHAIN, false, true, OutT>(a, stream);
        return edges ? launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, true, true, OutT>(a, stream)
                     : launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, false, true, OutT>(a, stream);
    }
    // Small graphs with the header-sized workspace the query asks for them:
    // the LDS walk.
    // (it stores single elements: no alignment needed)
    if (workspace_bytes >= kRecordOffset &&
        lds_walk_fits(w.num_nodes, w.num_edges, w.num_walks, w.walk_length)) {
        // (mlxc_rejection_sampling cleared the status words before this launch)
        N2VRecArgs a{};
        a.w = w;
        a.rows = p.rows;
        a.thr0 = float_at_or_above(p.prob0);
        a.thr1 = float_at_or_above(p.prob1);
        a.thr2 = float_at_or_above(p.prob2);
        a.key0 = p.key0;
        a.key1 = p.key1;
        // Every block copies the graph with all its threads, then walks with
        // some of them: at most one block per compute unit, and down to one
        // wavefront per SIMD (256 walking lanes) while the walks allow, since
        // the walk of a trial is bound by its own instruction latency (a
        // Philox draw per trial) once a SIMD has no other wavefront to run.
        // Each walk gets as many lanes (up to MLXC_LDS_MAX_GROUP) as keep its
        // call within one wavefront per SIMD of the device.
        DeviceInfo info;
        if (int rc = device_info(info)) return rc;
        const int64_t N = w.num_walks;  // 1 .. kLdsWalkSteps (lds_walk_fits)
        int G = 1;
        while (G < MLXC_LDS_MAX_GROUP && N * G * 2 <= static_cast<int64_t>(info.cus) * kLdsMinWalkers)
            G *= 2;
        const int64_t lanes = N * G;
        int64_t blocks = (lanes + kLdsMinWalkers - 1) / kLdsMinWalkers;
        if (blocks > info.cus) blocks = info.cus;
        if (blocks < 1) blocks = 1;
        int64_t threads = (lanes + blocks - 1) / blocks;
        threads = (threads + kWave - 1) / kWave * kWave;
        threads = threads < kLdsMinWalkers ? kLdsMinWalkers : threads > kLdsBlock ? kLdsBlock : threads;
        a.lds_group = G;
        a.lds_walkers = static_cast<int32_t>(threads / G);
        const dim3 grid(static_cast<unsigned>(blocks));
        const dim3 block(kLdsBlock);
        const bool edges = w.e_out != nullptr;
        if (int rc = record_walk_event(0, stream)) return rc;
        if (p.rule == MLXC_RULE_REF_CHAIN) {
            if (edges) hipLaunchKernelGGL((node2vec_lds_kernel<MLXC_RULE_REF_CHAIN, true, OutT>), grid, block, 0, stream, a);
            else hipLaunchKernelGGL((node2vec_lds_kernel<MLXC_RULE_REF_CHAIN, false, OutT>), grid, block, 0, stream, a);
        } else {
            if (edges) hipLaunchKernelGGL((node2vec_lds_kernel<MLXC_RULE_NODE2VEC_EXACT, true, OutT>), grid, block, 0, stream, a);
            else hipLaunchKernelGGL((node2vec_lds_kernel<MLXC_RULE_NODE2VEC_EXACT, false, OutT>), grid, block, 0, stream, a);
        }
        MLXC_HIP_TRY(hipGetLastError());
        return record_walk_event(1, stream);
    }
    // Graphs beyond int32, a workspace too small for the records, or output
    // buffers not 16-byte aligned: the direct CSR kernel.  The CSR check
    // validates the whole graph as the other layouts do; csr_status_kernel
    // turns its words into the call's status bits and the row order, on the
    // device.
    if (int rc = launch_csr_check(w.rowptr, w.num_nodes, w.col, w.num_edges, w.work, stream))
        return rc;
    if (int rc = launch_csr_status(w.work, stream)) return rc;
    N2VArgs a;
    a.w = w;
    a.prob0 = p.prob0;
    a.prob1 = p.prob1;
    a.prob2 = p.prob2;
    a.key0 = p.key0;
    a.key1 = p.key1;
    a.rows = p.rows;
    const bool edges = w.e_out != nullptr;
    return p.rule == MLXC_RULE_REF_CHAIN
               ? dispatch_n2v<MLXC_RULE_REF_CHAIN, OutT>(a, edges, stream)
               : dispatch_n2v<MLXC_RULE_NODE2VEC_EXACT, OutT>(a, edges, stream);
}

}  // namespace

int launch_node2vec(const WalkArgs& w, const N2VParams& p, void* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
    return p.out_type == MLXC_OUT_INT32
               ? launch_node2vec_typed<int32_t>(w, p, workspace, workspace_bytes, stream)
               : launch_node2vec_typed<int64_t>(w, p, workspace, workspace_bytes, stream);
}

}  // namespace mlxc
