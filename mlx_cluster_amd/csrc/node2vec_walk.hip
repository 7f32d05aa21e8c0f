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

// ------------------------------------------------------------- launcher

namespace {

template <int kRule, bool kSorted, bool kEdges>
int launch_n2v(const N2VArgs& a, hipStream_t stream) {
    auto kernel = node2vec_walk_kernel<kRule, kSorted, kEdges>;
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.w.num_walks, 1, grid)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

template <int kRule>
int dispatch_n2v(const N2VArgs& a, bool sorted, bool edges, hipStream_t stream) {
    if (sorted)
        return edges ? launch_n2v<kRule, true, true>(a, stream)
                     : launch_n2v<kRule, true, false>(a, stream);
    return edges ? launch_n2v<kRule, false, true>(a, stream)
                 : launch_n2v<kRule, false, false>(a, stream);
}

}  // namespace

size_t node2vec_workspace_bytes(int64_t, int64_t, int64_t, int32_t) {
    return MLXC_WORK_WORDS * sizeof(int64_t);
}

int launch_node2vec(const WalkArgs& w, const N2VParams& p, void*, size_t, hipStream_t stream) {
    N2VArgs a;
    a.w = w;
    a.prob0 = p.prob0;
    a.prob1 = p.prob1;
    a.prob2 = p.prob2;
    a.key0 = p.key0;
    a.key1 = p.key1;
    const bool edges = w.e_out != nullptr;
    return p.rule == MLXC_RULE_REF_CHAIN
               ? dispatch_n2v<MLXC_RULE_REF_CHAIN>(a, p.rows_sorted, edges, stream)
               : dispatch_n2v<MLXC_RULE_NODE2VEC_EXACT>(a, p.rows_sorted, edges, stream);
}

}  // namespace mlxc
