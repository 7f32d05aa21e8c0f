// Host evaluation of both walks: the stream="cpu" path of the reference
// (RandomWalk::eval_cpu, /root/reference/random_walks/RandomWalk.cpp:18-62;
// BiasedRandomWalk::eval_cpu, BiasedRandomWalk.cpp:30-102).  It produces the
// same outputs as the HIP kernels for the same inputs and seed: the same
// float32 index rule, Philox4x32-10 stream, FP64 acceptance constants, trial
// cap and handling of out-of-range values.  Walks are independent, so they
// are spread over std::threads in chunks taken from a shared counter.
#include <algorithm>
#include <atomic>
#include <exception>
#include <thread>
#include <vector>

#include "walk_host.h"

namespace mlxc {
namespace {

// Philox4x32-10, the generator of walk_device.h, with each high product word
// taken from a 64-bit multiply.
inline void philox_host(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3, uint32_t k0,
                        uint32_t k1) {
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = uint64_t{0xD2511F53u} * c0;
        const uint64_t p1 = uint64_t{0xCD9E8D57u} * c2;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        c0 = n0;
        c1 = static_cast<uint32_t>(p1);
        c2 = n2;
        c3 = static_cast<uint32_t>(p0);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

inline float unit_float_host(uint32_t x) { return static_cast<float>(x >> 8) * 0x1p-24f; }

// The float32 index rule of RandomWalk.cpp:51-53 with pick_index's clamp.
// The library is built with -ffp-contract=off, so r * fdeg is a single
// IEEE float32 multiply rounded to nearest, as __fmul_rn on the device.
inline int64_t pick_index_host(float r, int64_t deg) {
    if (deg <= (int64_t{1} << 24)) {
        const float fdeg = static_cast<float>(static_cast<int32_t>(deg));
        const float p = r * fdeg;
        if (!(p >= 0.0f)) return 0;
        if (p >= fdeg) return deg - 1;
        return static_cast<int64_t>(static_cast<int32_t>(p));
    }
    const float fdeg = static_cast<float>(deg);
    const float p = r * fdeg;
    if (!(p >= 0.0f)) return 0;
    if (p >= 9.0e18f) return deg - 1;
    const int64_t idx = static_cast<int64_t>(p);
    return idx < deg ? idx : deg - 1;
}

inline bool node_in(int64_t v, int64_t num_nodes) {
    return static_cast<uint64_t>(v) < static_cast<uint64_t>(num_nodes);
}

inline bool row_in(int64_t begin, int64_t end, int64_t num_edges) {
    return begin >= 0 && end >= begin && end <= num_edges;
}

// Runs body(first, last) -> status bits over [0, n) in chunks of `chunk`
// items on up to `threads` threads (the caller's thread is one of them) and
// returns the OR of the bits.
template <class Body>
int run_chunks(int64_t n, int threads, int64_t chunk, Body body, uint32_t& status) {
    status = 0;
    if (n <= 0) return MLXC_OK;
    const int64_t chunks = (n + chunk - 1) / chunk;
    const int workers = static_cast<int>(std::min<int64_t>(std::max(threads, 1), chunks));
    std::atomic<int64_t> next{0};
    std::atomic<uint32_t> bits{0};
    auto worker = [&]() {
        uint32_t local = 0;
        for (;;) {
            const int64_t c = next.fetch_add(1, std::memory_order_relaxed);
            if (c >= chunks) break;
            const int64_t first = c * chunk;
            local |= body(first, std::min(n, first + chunk));
        }
        bits.fetch_or(local, std::memory_order_relaxed);
    };
    std::vector<std::thread> pool;
    try {
        pool.reserve(workers - 1);
        for (int i = 1; i < workers; ++i) pool.emplace_back(worker);
    } catch (const std::exception&) {
        // No more threads: the ones that started and this one take every chunk.
    }
    worker();
    for (auto& t : pool) t.join();
    status = bits.load();
    return MLXC_OK;
}

int resolve_threads(int32_t threads) {
    if (threads > 0) return threads;
    const unsigned hw = std::thread::hardware_concurrency();
    return hw ? static_cast<int>(hw) : 1;
}

constexpr int64_t kHostChunk = 1024;  // walks per chunk

// Threads worth starting for a call of `steps` walk steps: starting one costs
// tens of microseconds, as much as ~3,000 uniform steps, so small calls (the
// reference tests' 2,000 walks of 5 steps) run on fewer threads than allowed.
// Measured on an 8-core host with the Cora-like graph: a uniform call of
// 10,000 steps 127 us on one thread against 180 us on eight; a node2vec call
// of 10,000 steps (about 18,000 trials and linear row scans) 700 us on two
// against 1,000 us on one.
constexpr int64_t kUniformStepsPerThread = int64_t{1} << 16;
constexpr int64_t kNode2vecStepsPerThread = int64_t{1} << 12;
int threads_for(int allowed, int64_t steps, int64_t steps_per_thread) {
    const int64_t useful = steps / steps_per_thread;
    return useful < 1 ? 1 : useful < allowed ? static_cast<int>(useful) : allowed;
}

// Uniform walks [first, last): the loop of RandomWalk.cpp:41-60, with the
// out-of-range handling of uniform_walk_kernel (the walk stops and repeats
// its node, edge id -1).
template <bool kGen, typename OutT>
uint32_t uniform_range(const HostWalk& w, int64_t first, int64_t last) {
    const int64_t L = w.walk_length;
    uint32_t status = 0;
    for (int64_t n = first; n < last; ++n) {
        OutT* out = static_cast<OutT*>(w.n_out) + n * (L + 1);
        OutT* eout = w.e_out ? static_cast<OutT*>(w.e_out) + n * L : nullptr;
        int64_t v = w.start[n];
        out[0] = static_cast<OutT>(v);
        int64_t l = 0;
        int64_t block = -1;  // Philox block whose four uniforms are in u[]
        float u[4] = {0.f, 0.f, 0.f, 0.f};
        if (!node_in(v, w.num_nodes)) {
            status |= MLXC_STATUS_BAD_NODE;
        } else {
            for (; l < L; ++l) {
                const int64_t begin = w.rowptr[v], end = w.rowptr[v + 1];
                if (!row_in(begin, end, w.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                    break;
                }
                if (end == begin) break;  // out-degree 0: the walk stays here
                const int64_t i = n * L + l;
                float r;
                if (kGen) {
                    const int64_t g = (w.walk_base + n) * L + l;  // stream position
                    if ((g >> 2) != block) {
                        block = g >> 2;
                        uint32_t c0 = static_cast<uint32_t>(block);
                        uint32_t c1 = static_cast<uint32_t>(static_cast<uint64_t>(block) >> 32);
                        uint32_t c2 = 0, c3 = 0;
                        philox_host(c0, c1, c2, c3, w.key0, w.key1);
                        u[0] = unit_float_host(c0);
                        u[1] = unit_float_host(c1);
                        u[2] = unit_float_host(c2);
                        u[3] = unit_float_host(c3);
                    }
                    r = u[g & 3];
                } else {
                    r = w.rand[i];
                }
                const int64_t e = begin + pick_index_host(r, end - begin);
                const int64_t x = w.col[e];
                out[l + 1] = static_cast<OutT>(x);
                if (eout) eout[l] = static_cast<OutT>(e);
                v = x;
                if (!node_in(x, w.num_nodes)) {
                    status |= MLXC_STATUS_BAD_NODE;
                    ++l;
                    break;
                }
            }
        }
        for (int64_t j = l; j < L; ++j) {
            out[j + 1] = static_cast<OutT>(v);
            if (eout) eout[j] = -1;
        }
    }
    return status;
}

// t in row(x)?  BiasedRandomWalk.cpp:20-28 scans the row; sorted rows are
// bisected with the same answer.
bool is_neighbor_host(const HostWalk& w, bool sorted, int64_t x, int64_t t, uint32_t& status) {
    const int64_t begin = w.rowptr[x], end = w.rowptr[x + 1];
    if (!row_in(begin, end, w.num_edges)) {
        status |= MLXC_STATUS_BAD_ROW;
        return false;
    }
    if (!sorted) return std::find(w.col + begin, w.col + end, t) != w.col + end;
    const int64_t* it = std::lower_bound(w.col + begin, w.col + end, t);
    return it != w.col + end && *it == t;
}

template <int kRule>
bool accept_host(const HostWalk& w, const N2VParams& prm, bool sorted, double r, int64_t x,
                 int64_t t, uint32_t& status) {
    if (kRule == MLXC_RULE_REF_CHAIN) {  // BiasedRandomWalk.cpp:86-91, side-effect free
        if (r < prm.prob2) return true;
        if (x == t && r < prm.prob0) return true;
        if (r < prm.prob1) return is_neighbor_host(w, sorted, x, t, status);
        return false;
    }
    if (x == t) return r < prm.prob0;
    const bool lt1 = r < prm.prob1, lt2 = r < prm.prob2;
    if (lt1 && lt2) return true;
    if (!lt1 && !lt2) return false;
    return is_neighbor_host(w, sorted, x, t, status) ? lt1 : lt2;
}

// node2vec walks [first, last): BiasedRandomWalk.cpp:57-100 on the Philox
// stream (counter = walk, step, trial), as node2vec_walk_kernel.
template <int kRule, typename OutT>
uint32_t node2vec_range(const HostWalk& w, const N2VParams& prm, bool sorted, int64_t first,
                        int64_t last) {
    const int64_t L = w.walk_length;
    const int64_t V = w.num_nodes;
    uint32_t status = 0;
    for (int64_t n = first; n < last; ++n) {
        OutT* out = static_cast<OutT*>(w.n_out) + n * (L + 1);
        OutT* eout = w.e_out ? static_cast<OutT*>(w.e_out) + n * L : nullptr;
        int64_t t = w.start[n];
        out[0] = static_cast<OutT>(t);
        if (L == 0) {
            if (!node_in(t, V)) status |= MLXC_STATUS_BAD_NODE;
            continue;
        }
        const uint64_t sn = static_cast<uint64_t>(w.walk_base + n);  // Philox stream index
        const uint32_t n_lo = static_cast<uint32_t>(sn);
        const uint32_t n_hi = static_cast<uint32_t>(sn >> 32);
        bool bad = !node_in(t, V);
        int64_t v = t, e = -1;
        if (bad) {
            status |= MLXC_STATUS_BAD_NODE;
        } else {
            // First step: uniform, no acceptance test (BiasedRandomWalk.cpp:60-66).
            const int64_t begin = w.rowptr[t], end = w.rowptr[t + 1];
            if (!row_in(begin, end, w.num_edges)) {
                status |= MLXC_STATUS_BAD_ROW;
                bad = true;
            } else if (end > begin) {
                uint32_t c0 = n_lo, c1 = n_hi, c2 = 0, c3 = 0;
                philox_host(c0, c1, c2, c3, prm.key0, prm.key1);
                e = begin + pick_index_host(unit_float_host(c0), end - begin);
                v = w.col[e];
            }
        }
        out[1] = static_cast<OutT>(v);
        if (eout) eout[0] = static_cast<OutT>(e);
        for (int64_t l = 1; l < L; ++l) {
            int64_t x = v;
            e = -1;
            if (!bad && !node_in(v, V)) {
                status |= MLXC_STATUS_BAD_NODE;
                bad = true;
            }
            if (!bad) {
                const int64_t begin = w.rowptr[v], end = w.rowptr[v + 1];
                const int64_t deg = end - begin;
                if (!row_in(begin, end, w.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                    bad = true;
                } else if (deg == 1) {  // BiasedRandomWalk.cpp:76-78: forced, no draw
                    e = begin;
                    x = w.col[e];
                } else if (deg > 1) {  // :80-92, capped at MLXC_MAX_TRIALS
                    for (uint32_t trial = 0;; ++trial) {
                        uint32_t c0 = n_lo, c1 = n_hi, c2 = static_cast<uint32_t>(l), c3 = trial;
                        philox_host(c0, c1, c2, c3, prm.key0, prm.key1);
                        e = begin + pick_index_host(unit_float_host(c0), deg);
                        x = w.col[e];
                        const double r = static_cast<double>(unit_float_host(c1));
                        if (!node_in(x, V)) {
                            status |= MLXC_STATUS_BAD_NODE;
                            bad = true;
                            break;
                        }
                        if (accept_host<kRule>(w, prm, sorted, r, x, t, status)) break;
                        if (trial + 1 >= MLXC_MAX_TRIALS) break;
                    }
                }
            }
            out[l + 1] = static_cast<OutT>(x);
            if (eout) eout[l] = static_cast<OutT>(e);
            t = v;
            v = x;
        }
    }
    return status;
}

// CSR validation as the device preparation pass (edge_record_kernel) does it:
// BAD_NODE for a col value outside [0, V), BAD_ROW for rowptr[0] != 0,
// rowptr[V] != E or a decreasing rowptr; rows are sorted iff every descent
// col[i] < col[i-1] sits at the start of a non-empty row.
uint32_t host_csr_scan(const HostWalk& w, int threads, bool& sorted) {
    const int64_t V = w.num_nodes, E = w.num_edges;
    std::atomic<int64_t> desc{0}, start_desc{0};
    uint32_t col_bits = 0, row_bits = 0;
    run_chunks(E, threads, int64_t{1} << 16, [&](int64_t first, int64_t last) -> uint32_t {
        uint32_t s = 0;
        int64_t d = 0;
        for (int64_t i = first; i < last; ++i) {
            const int64_t c = w.col[i];
            if (!node_in(c, V)) s = MLXC_STATUS_BAD_NODE;
            if (i >= 1 && c < w.col[i - 1]) ++d;
        }
        desc.fetch_add(d, std::memory_order_relaxed);
        return s;
    }, col_bits);
    run_chunks(V, threads, int64_t{1} << 16, [&](int64_t first, int64_t last) -> uint32_t {
        uint32_t s = 0;
        int64_t d = 0;
        for (int64_t v = first; v < last; ++v) {
            const int64_t rs = w.rowptr[v], re = w.rowptr[v + 1];
            if (re < rs) s = MLXC_STATUS_BAD_ROW;
            if (rs >= 1 && re > rs && re <= E && w.col[rs] < w.col[rs - 1]) ++d;
        }
        start_desc.fetch_add(d, std::memory_order_relaxed);
        return s;
    }, row_bits);
    uint32_t status = col_bits | row_bits;
    if (w.rowptr[0] != 0 || w.rowptr[V] != E) status |= MLXC_STATUS_BAD_ROW;
    sorted = desc.load() == start_desc.load();
    return status;
}

template <typename OutT>
int host_uniform_typed(const HostWalk& w, bool generate, int t, uint32_t& status) {
    if (generate)
        return run_chunks(w.num_walks, t, kHostChunk,
                          [&](int64_t a, int64_t b) { return uniform_range<true, OutT>(w, a, b); },
                          status);
    return run_chunks(w.num_walks, t, kHostChunk,
                      [&](int64_t a, int64_t b) { return uniform_range<false, OutT>(w, a, b); },
                      status);
}

template <typename OutT>
int host_node2vec_typed(const HostWalk& w, const N2VParams& prm, bool sorted, int t,
                        uint32_t& status) {
    if (prm.rule == MLXC_RULE_REF_CHAIN)
        return run_chunks(w.num_walks, t, kHostChunk, [&](int64_t a, int64_t b) {
            return node2vec_range<MLXC_RULE_REF_CHAIN, OutT>(w, prm, sorted, a, b);
        }, status);
    return run_chunks(w.num_walks, t, kHostChunk, [&](int64_t a, int64_t b) {
        return node2vec_range<MLXC_RULE_NODE2VEC_EXACT, OutT>(w, prm, sorted, a, b);
    }, status);
}

}  // namespace

namespace {

template <typename T>
void windows_of(const T* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx, T* out) {
    const int64_t windows = walk_nodes - ctx + 1;
    for (int64_t j = 0; j < windows; ++j)
        for (int64_t n = 0; n < num_walks; ++n)
            for (int32_t k = 0; k < ctx; ++k)
                out[(j * num_walks + n) * ctx + k] = walks[n * walk_nodes + j + k];
}

template <typename T>
void negative_windows_of(const int64_t* start, int64_t num_walks, int32_t walk_length,
                         int32_t ctx, int64_t num_nodes, uint64_t seed, T* out) {
    const int32_t walk_nodes = walk_length + 1;
    std::vector<T> rw(static_cast<size_t>(num_walks) * walk_nodes);
    for (int64_t n = 0; n < num_walks; ++n) {
        rw[n * walk_nodes] = static_cast<T>(start[n]);
        for (int32_t l = 1; l < walk_nodes; ++l) {
            uint32_t c0 = static_cast<uint32_t>(n), c1 = static_cast<uint32_t>(
                                                        static_cast<uint64_t>(n) >> 32),
                     c2 = static_cast<uint32_t>(l), c3 = 0;
            philox_host(c0, c1, c2, c3, static_cast<uint32_t>(seed),
                        static_cast<uint32_t>(seed >> 32));
            rw[n * walk_nodes + l] = static_cast<T>(
                (static_cast<uint64_t>(c0) * static_cast<uint64_t>(num_nodes)) >> 32);
        }
    }
    windows_of(rw.data(), num_walks, walk_nodes, ctx, out);
}

}  // namespace

void host_context_windows(const void* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                          int32_t elem_type, void* out) {
    if (elem_type == MLXC_OUT_INT32)
        windows_of(static_cast<const int32_t*>(walks), num_walks, walk_nodes, ctx,
                   static_cast<int32_t*>(out));
    else
        windows_of(static_cast<const int64_t*>(walks), num_walks, walk_nodes, ctx,
                   static_cast<int64_t*>(out));
}

void host_negative_windows(const int64_t* start, int64_t num_walks, int32_t walk_length,
                           int32_t ctx, int64_t num_nodes, uint64_t seed, int32_t out_type,
                           void* out) {
    if (out_type == MLXC_OUT_INT32)
        negative_windows_of(start, num_walks, walk_length, ctx, num_nodes, seed,
                            static_cast<int32_t*>(out));
    else
        negative_windows_of(start, num_walks, walk_length, ctx, num_nodes, seed,
                            static_cast<int64_t*>(out));
}

int host_uniform(const HostWalk& w, bool generate, int32_t threads, uint32_t& status) {
    const int t = threads_for(resolve_threads(threads), w.num_walks * w.walk_length,
                              kUniformStepsPerThread);
    return w.out_type == MLXC_OUT_INT32 ? host_uniform_typed<int32_t>(w, generate, t, status)
                                        : host_uniform_typed<int64_t>(w, generate, t, status);
}

int host_node2vec(const HostWalk& w, const N2VParams& prm, int32_t threads, uint32_t& status) {
    const int all = resolve_threads(threads);
    const int t = threads_for(all, w.num_walks * w.walk_length, kNode2vecStepsPerThread);
    // the whole CSR is validated on every call, as the device layouts do (its
    // chunks of 2^16 entries set how many of the threads it uses)
    uint32_t prep = 0;
    bool sorted = prm.rows == MLXC_ROWS_SORTED;
    if (w.num_walks > 0) {
        bool detected = false;
        prep = host_csr_scan(w, all, detected);
        if (prm.rows == MLXC_ROWS_DETECT) sorted = detected;
    }
    const int rc = w.out_type == MLXC_OUT_INT32
                       ? host_node2vec_typed<int32_t>(w, prm, sorted, t, status)
                       : host_node2vec_typed<int64_t>(w, prm, sorted, t, status);
    status |= prep;
    return rc;
}

}  // namespace mlxc
