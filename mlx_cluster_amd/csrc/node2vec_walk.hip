// node2vec walk by rejection sampling (BiasedRandomWalk.cpp:52-100) and its
// launcher.  The reference has no GPU version (BiasedRandomWalk.cpp:150-155).
#include "walk_host.h"

namespace mlxc {

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

template <int kRule, bool kSorted, bool kEdges, typename OutT>
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
        OutT* out = static_cast<OutT*>(a.w.n_out) + n * (L + 1);
        OutT* eout = kEdges ? static_cast<OutT*>(a.w.e_out) + n * L : nullptr;
        int64_t t = a.w.start[n];
        out[0] = static_cast<OutT>(t);
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
        out[1] = static_cast<OutT>(v);
        if (kEdges) eout[0] = static_cast<OutT>(e);
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
            out[l + 1] = static_cast<OutT>(x);
            if (kEdges) eout[l] = static_cast<OutT>(e);
            t = v;
            v = x;
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// ---------------------------------------------------- record node2vec walk

// Slot phases of the record walk.
enum : int {
    kN2vIdle = 0,    // wants a walk id
    kN2vStart = 1,   // reads the start record of walk n
    kN2vCand = 2,     // reads the edge record of the current candidate
    kN2vSummary = 3,  // sorted rows: bisects the block index of row(x)
    kN2vBlock = 4,    // sorted rows: reads the 16-entry block that may hold t
    kN2vScan = 5,     // unsorted rows: reads the next entry of row(x)
    kN2vDone = 6,     // the queue is exhausted
};

// The two uniforms of a trial: Philox4x32-10 with key = seed and counter =
// (walk lo, walk hi, step, trial); word 0 picks the candidate, word 1 is
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

// Neighbour search on sorted rows.  col32 is col as int32 (padded to a
// multiple of kSearchBlock entries) and index[j] = col32[kSearchBlock * j]:
// a dense sample of every row, E / 16 entries, that stays in the caches.  A
// search bisects the index entries inside row(x) and then reads the one
// aligned 64-byte block of col32 that can hold t — one line from HBM instead
// of one per bisection step.
constexpr int kSearchBlock = 16;

struct N2VRecArgs {
    WalkArgs w;
    const EdgeRecord* recs;   // [num_edges]
    const EdgeRecord* init;   // [num_walks]
    const int32_t* col32;     // [num_edges rounded up to kSearchBlock] col as int32
    const int32_t* index;     // [ceil(num_edges / kSearchBlock)] col32[kSearchBlock * j]
    int32_t rows;             // MLXC_ROWS_*; DETECT reads the prep pass's counts in work[2..3]
    double prob0, prob1, prob2;
    uint32_t key0, key1;
};

// Decision on candidate x for r before any row search: 1 accept, 0 reject,
// -1 the answer depends on whether t is in row(x).  The reference's chain
// (BiasedRandomWalk.cpp:86-91: (x==t && r<p0) || (nb(x,t) && r<p1) || r<p2)
// has no side effects, so its cheap terms decide first; the analytic rule
// uses p0 when x == t, else p1 or p2 by adjacency.
template <int kRule>
__device__ __forceinline__ int n2v_decide(const N2VRecArgs& a, double r, int32_t x, int32_t t) {
    if (kRule == MLXC_RULE_REF_CHAIN) {
        if (r < a.prob2) return 1;
        if (x == t && r < a.prob0) return 1;
        return r < a.prob1 ? -1 : 0;
    }
    if (x == t) return r < a.prob0 ? 1 : 0;
    const bool lt1 = r < a.prob1, lt2 = r < a.prob2;
    if (lt1 && lt2) return 1;
    if (!lt1 && !lt2) return 0;
    return -1;
}

// Decision once the search has answered whether t is in row(x).
template <int kRule>
__device__ __forceinline__ bool n2v_resolve(const N2VRecArgs& a, double r, bool adjacent) {
    if (kRule == MLXC_RULE_REF_CHAIN) return adjacent;  // only searched when r < p1 decides
    return adjacent ? (r < a.prob1) : (r < a.prob2);
}

// node2vec walk over edge records (num_nodes, num_edges below 2^31; n_out and
// e_out 16-byte aligned).  One walk per lane slot from the wave queue.  Every iteration a
// live slot issues one dependent read — a start record, the edge record of
// its candidate (which carries the candidate's row, so the neighbour test
// needs no rowptr read), or one step of the neighbour search — and the wave
// waits once.  Sorted rows are searched through the block index (see
// kSearchBlock); unsorted rows are scanned one entry per iteration, as the
// reference scans them.
template <int kRule, bool kEdges, typename OutT>
__global__ __launch_bounds__(kBlock) void node2vec_rec_kernel(N2VRecArgs a) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    OutT* const nout = static_cast<OutT*>(a.w.n_out);
    OutT* const eout = static_cast<OutT*>(a.w.e_out);
    const bool sorted = a.rows == MLXC_ROWS_SORTED ||
                        (a.rows == MLXC_ROWS_DETECT && a.w.work[2] == a.w.work[3]);
    const int64_t L = a.w.walk_length;
    const int64_t L1 = L + 1;
    const int64_t N = a.w.num_walks;
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.w.work + 1);
    WaveQueue q{0, 0};
    int phase = kN2vIdle;
    int64_t n = 0;
    int32_t l = 0;          // steps done
    uint32_t trial = 0;
    int32_t t = 0;          // previous node
    int32_t v = 0, bv = 0, dv = 0;   // current node and its row
    int32_t e = 0;          // candidate edge
    int32_t x = 0, bx = 0, dx = 0;   // candidate node and its row (from its record)
    int32_t lo = 0, hi = 0; // search range: index entries (sorted) or col32 entries (unsorted)
    int32_t first = 0;      // first index entry inside row(x)
    int32_t blk = 0, blo = 0, bhi = 0;  // block to read and the row's entries in it
    float r = 0.0f;         // acceptance uniform of the current trial
    OutWin<int32_t> ow;
    OutWin<int32_t> ew;     // edge ids (kEdges): e_out[n*L + l] is step l's edge
    ow_init(ow);
    ow_init(ew);
    __shared__ WaveStage stage[kBlock / kWave];
    WaveStage& st = stage[threadIdx.x / kWave];
    uint32_t status = 0;

    while (true) {
        // 1. This iteration's read: a record, an index entry, a block of
        // col32 or one col32 entry.
        const int ph = phase;
        const EdgeRecord* p = ph == kN2vStart ? a.init + n : ph == kN2vCand ? a.recs + e : a.init;
        const i32x4 rec = *reinterpret_cast<const i32x4*>(p);
        const int32_t mid = lo + ((hi - lo) >> 1);
        int32_t sv;                       // kN2vSummary / kN2vScan
        i32x4 blkv[kSearchBlock / 4];    // kN2vBlock
        if (ph == kN2vSummary) sv = a.index[mid];
        if (ph == kN2vScan) sv = a.col32[lo];
        if (ph == kN2vBlock) {
            const i32x4* bp = reinterpret_cast<const i32x4*>(a.col32 + kSearchBlock * blk);
#pragma unroll
            for (int i = 0; i < kSearchBlock / 4; ++i) blkv[i] = bp[i];
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
            phase = id < N ? kN2vStart : kN2vDone;
        }
        if (!__any(phase != kN2vDone)) break;
        wait_vmem();
        keep_vgpr(rec.w);
        if (ph == kN2vIdle || ph == kN2vDone) continue;

        // 3. Consume.
        const int64_t g0 = n * L1;
        const int64_t e0 = n * L;  // edge output index of the walk's step 0
        bool push = false, fill = false, flush = false, accept = false, next_trial = false;
        int64_t g = g0 + l;  // output index of the last buffered entry
        if (ph == kN2vStart) {
            ow.count = 0;
            ew.count = 0;
            v = rec.x;
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
                float u0;
                n2v_uniforms(n, 0, 0u, a.key0, a.key1, u0, r);
                e = bv + static_cast<int32_t>(pick_index(u0, dv));
                trial = 0;
                phase = kN2vCand;
            }
        } else if (ph == kN2vCand) {
            x = rec.x;
            bx = rec.y;
            dx = rec.z;
            if (dx < 0) {
                status |= dx == kRecBadNode ? MLXC_STATUS_BAD_NODE : MLXC_STATUS_BAD_ROW;
                fill = true;
            } else if (l == 0 || dv == 1) {
                accept = true;  // first step, or a forced step (BiasedRandomWalk.cpp:76-78)
            } else {
                const int d = n2v_decide<kRule>(a, static_cast<double>(r), x, t);
                if (d == 1) {
                    accept = true;
                } else if (d == 0) {
                    next_trial = true;
                } else if (dx == 0) {
                    accept = n2v_resolve<kRule>(a, static_cast<double>(r), false);
                    next_trial = !accept;
                } else if (!sorted) {
                    lo = bx;
                    hi = bx + dx;
                    phase = kN2vScan;
                } else {
                    // index entries j with bx <= kSearchBlock * j < bx + dx
                    first = (bx + kSearchBlock - 1) / kSearchBlock;
                    const int32_t last = (bx + dx - 1) / kSearchBlock;
                    if (first > last) {  // short row inside one block
                        blk = bx / kSearchBlock;
                        blo = bx;
                        bhi = bx + dx;
                        phase = kN2vBlock;
                    } else {
                        lo = first;
                        hi = last + 1;
                        phase = kN2vSummary;
                    }
                }
            }
        } else {  // the neighbour search: is t in row(x)?
            bool done = false, found = false;
            if (ph == kN2vSummary) {
                if (sv == t) {
                    done = found = true;
                } else {
                    if (sv < t) lo = mid + 1;
                    else hi = mid;
                    if (lo >= hi) {
                        // index entries first .. lo-1 are < t, lo .. are > t:
                        // t can only be in the block after entry lo-1, or
                        // before the row's first index entry
                        const int32_t row_end = bx + dx;
                        if (lo == first) {
                            blk = first - 1;
                            blo = bx;
                            bhi = min(kSearchBlock * first, row_end);
                        } else {
                            blk = lo - 1;
                            blo = kSearchBlock * blk;
                            bhi = min(blo + kSearchBlock, row_end);
                        }
                        phase = kN2vBlock;
                    }
                }
            } else if (ph == kN2vBlock) {
#pragma unroll
                for (int i = 0; i < kSearchBlock; ++i) {
                    const int32_t idx = kSearchBlock * blk + i;
                    const int32_t cv = blkv[i / 4][i % 4];
                    found |= idx >= blo && idx < bhi && cv == t;
                }
                done = true;
            } else {  // kN2vScan
                if (sv == t) {
                    done = found = true;
                } else {
                    lo += 1;
                    done = lo >= hi;
                }
            }
            if (done) {
                accept = n2v_resolve<kRule>(a, static_cast<double>(r), found);
                next_trial = !accept;
            }
        }
        if (next_trial) {
            trial += 1;
            if (trial >= MLXC_MAX_TRIALS) {
                accept = true;  // trial cap: keep the last candidate
            } else {
                float u0;
                n2v_uniforms(n, l, trial, a.key0, a.key1, u0, r);
                e = bv + static_cast<int32_t>(pick_index(u0, dv));
                phase = kN2vCand;
            }
        }
        if (accept) {
            if (kEdges) ow_push(ew, eout, e0 + l, e);
            push = true;
            g += 1;
            l += 1;
            t = v;
            v = x;
            bv = bx;
            dv = dx;
            if (l == L) {
                flush = true;
            } else if (dv == 0) {
                fill = true;
            } else {
                trial = 0;
                if (dv == 1) {
                    e = bv;  // forced: no draw
                } else {
                    float u0;
                    n2v_uniforms(n, l, 0u, a.key0, a.key1, u0, r);
                    e = bv + static_cast<int32_t>(pick_index(u0, dv));
                }
                phase = kN2vCand;
            }
        }
        if (push) ow_push(ow, nout, g, v);
        if (fill) {
            ow_fill(ow, nout, g + 1, g0 + L, v);
            if (kEdges) ow_fill(ew, eout, e0 + l, e0 + L - 1, -1);  // l edges buffered
        } else if (flush) {
            if (ow.count) ow_flush(ow, nout, g);
            if (kEdges && ew.count) ow_flush(ew, eout, e0 + L - 1);
        }
        if (fill || flush) phase = kN2vIdle;
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.w.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------------------------- launcher

namespace {

template <int kRule, bool kSorted, bool kEdges, typename OutT>
int launch_n2v(const N2VArgs& a, hipStream_t stream) {
    auto kernel = node2vec_walk_kernel<kRule, kSorted, kEdges, OutT>;
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

template <int kRule, typename OutT>
int dispatch_n2v(const N2VArgs& a, bool sorted, bool edges, hipStream_t stream) {
    if (sorted)
        return edges ? launch_n2v<kRule, true, true, OutT>(a, stream)
                     : launch_n2v<kRule, true, false, OutT>(a, stream);
    return edges ? launch_n2v<kRule, false, true, OutT>(a, stream)
                 : launch_n2v<kRule, false, false, OutT>(a, stream);
}

// Resident blocks per compute unit of the node2vec record walk (0: as many
// as its registers allow, 5; fewer measured slower at configuration 3).
#ifndef MLXC_N2V_BLOCKS_PER_CU
#define MLXC_N2V_BLOCKS_PER_CU 0
#endif

template <int kRule, bool kEdges, typename OutT>
int launch_n2v_rec(const N2VRecArgs& a, hipStream_t stream) {
    auto kernel = node2vec_rec_kernel<kRule, kEdges, OutT>;
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid, MLXC_N2V_BLOCKS_PER_CU)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

// Workspace of the record walk: edge records, start records, then (128-byte
// aligned) col as int32 padded to whole search blocks, then the block index.
struct N2VLayout {
    size_t col32, index, total;
};

N2VLayout n2v_layout(int64_t num_edges, int64_t num_walks) {
    N2VLayout lay;
    const size_t blocks = static_cast<size_t>((num_edges + kSearchBlock - 1) / kSearchBlock);
    lay.col32 = kRecordOffset + static_cast<size_t>(num_edges + num_walks) * sizeof(EdgeRecord);
    lay.col32 = (lay.col32 + 127) & ~static_cast<size_t>(127);
    lay.index = lay.col32 + blocks * kSearchBlock * sizeof(int32_t);
    lay.total = lay.index + blocks * sizeof(int32_t);
    return lay;
}

}  // namespace

size_t node2vec_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                                int32_t walk_length) {
    if (num_nodes < 0 || num_edges < 0 || num_walks < 0 || walk_length < 0 ||
        !records_fit(num_nodes, num_edges))
        return MLXC_WORK_WORDS * sizeof(int64_t);
    return n2v_layout(num_edges, num_walks).total;
}

namespace {

template <typename OutT>
int launch_node2vec_typed(const WalkArgs& w, const N2VParams& p, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    const N2VLayout lay = n2v_layout(w.num_edges, w.num_walks);
    const bool aligned = reinterpret_cast<uintptr_t>(w.n_out) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(w.e_out) % 16 == 0;  // e_out may be null
    if (aligned && records_fit(w.num_nodes, w.num_edges) && workspace_bytes >= lay.total) {
        N2VRecArgs a;
        a.w = w;
        char* base = static_cast<char*>(workspace);
        EdgeRecord* recs = reinterpret_cast<EdgeRecord*>(base + kRecordOffset);
        EdgeRecord* init = recs + w.num_edges;
        int32_t* col32 = reinterpret_cast<int32_t*>(base + lay.col32);
        int32_t* index = reinterpret_cast<int32_t*>(base + lay.index);
        // one pass builds the search arrays and, for MLXC_ROWS_DETECT, checks
        // the rows (the walk reads the result on the device: no host sync)
        if (int rc = launch_edge_records(w.rowptr, w.col, w.num_nodes, w.num_edges, recs, col32,
                                         index, kSearchBlock,
                                         p.rows == MLXC_ROWS_DETECT ? w.work : nullptr, stream))
            return rc;
        if (int rc = launch_walk_init(w.rowptr, w.start, w.num_nodes, w.num_edges, w.num_walks,
                                      init, stream))
            return rc;
        a.recs = recs;
        a.init = init;
        a.col32 = col32;
        a.index = index;
        a.prob0 = p.prob0;
        a.prob1 = p.prob1;
        a.prob2 = p.prob2;
        a.key0 = p.key0;
        a.key1 = p.key1;
        a.rows = p.rows;
        const bool edges = w.e_out != nullptr;
        if (p.rule == MLXC_RULE_REF_CHAIN)
            return edges ? launch_n2v_rec<MLXC_RULE_REF_CHAIN, true, OutT>(a, stream)
                         : launch_n2v_rec<MLXC_RULE_REF_CHAIN, false, OutT>(a, stream);
        return edges ? launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, true, OutT>(a, stream)
                     : launch_n2v_rec<MLXC_RULE_NODE2VEC_EXACT, false, OutT>(a, stream);
    }
    // Graphs beyond int32, a workspace too small for the records, or output
    // buffers not 16-byte aligned: the direct CSR kernel, which needs the row
    // order on the host.
    bool sorted = p.rows == MLXC_ROWS_SORTED;
    if (p.rows == MLXC_ROWS_DETECT) {
        if (int rc = launch_csr_check(w.rowptr, w.num_nodes, w.col, w.num_edges, w.work, stream))
            return rc;
        int64_t host[3] = {0, 0, 0};
        MLXC_HIP_TRY(hipMemcpyAsync(host, w.work, sizeof(host), hipMemcpyDeviceToHost, stream));
        MLXC_HIP_TRY(hipStreamSynchronize(stream));
        if (host[0] & MLXC_CSR_BAD_ROWPTR) return fail(MLXC_ERR_INVALID_ARGUMENT, "rowptr is malformed");
        if (host[0] & MLXC_CSR_BAD_COL)
            return fail(MLXC_ERR_INVALID_ARGUMENT, "a col entry is outside [0, num_nodes)");
        sorted = host[1] == host[2];
        if (int rc = launch_zero_work(w.work, stream)) return rc;
    }
    N2VArgs a;
    a.w = w;
    a.prob0 = p.prob0;
    a.prob1 = p.prob1;
    a.prob2 = p.prob2;
    a.key0 = p.key0;
    a.key1 = p.key1;
    const bool edges = w.e_out != nullptr;
    return p.rule == MLXC_RULE_REF_CHAIN
               ? dispatch_n2v<MLXC_RULE_REF_CHAIN, OutT>(a, sorted, edges, stream)
               : dispatch_n2v<MLXC_RULE_NODE2VEC_EXACT, OutT>(a, sorted, edges, stream);
}

}  // namespace

int launch_node2vec(const WalkArgs& w, const N2VParams& p, void* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
    return p.out_type == MLXC_OUT_INT32
               ? launch_node2vec_typed<int32_t>(w, p, workspace, workspace_bytes, stream)
               : launch_node2vec_typed<int64_t>(w, p, workspace, workspace_bytes, stream);
}

}  // namespace mlxc
