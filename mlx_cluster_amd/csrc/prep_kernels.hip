// Per-call preparation kernels: workspace reset, edge records, start
// records, CSR validation and seeded uniform fills.
#include "walk_host.h"

namespace mlxc {

__global__ void zero_words_kernel(int64_t* p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ void copy_word_kernel(const int64_t* src, int64_t* dst) {
    if (threadIdx.x == 0) *dst = *src;
}

__device__ __forceinline__ int64_t wave_sum(int64_t x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

__device__ __forceinline__ uint32_t wave_or(uint32_t x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x |= __shfl_xor(x, off, kWave);
    return x;
}

// CSR validation, accumulated per thread and reduced per block.  Rows are
// sorted iff every position i >= 1 with col[i] < col[i-1] starts a non-empty
// row, i.e. iff desc == start_desc.
struct CsrCheck {
    bool bad_rowptr = false;  // rowptr[0] != 0, rowptr[V] != E, or decreasing
    bool bad_col = false;     // a col value outside [0, V)
    int64_t desc = 0;
    int64_t start_desc = 0;

    // node-parallel part: thread gid of a grid of `stride` threads
    __device__ void nodes(const int64_t* rowptr, int64_t V, const int64_t* col, int64_t E,
                          int64_t gid, int64_t stride) {
        if (gid == 0 && (rowptr[0] != 0 || rowptr[V] != E)) bad_rowptr = true;
        for (int64_t v = gid; v < V; v += stride) {
            const int64_t rs = rowptr[v], re = rowptr[v + 1];
            if (re < rs) bad_rowptr = true;
            if (rs >= 1 && re > rs && re <= E && col[rs] < col[rs - 1]) ++start_desc;
        }
    }
    // edge-parallel part: entry i holding c
    __device__ void edge(const int64_t* col, int64_t V, int64_t i, int64_t c) {
        if (!node_ok(c, V)) bad_col = true;
        if (i >= 1 && c < col[i - 1]) ++desc;
    }
    // Adds the block's totals to the given words, one atomic each from
    // thread 0: the status bits, and the descents that start no row
    // (desc - start_desc, zero exactly when the rows are sorted) to
    // diff_word.  Every thread of the block calls it.  (Atomics on one word
    // serialize: three per wavefront, 49,000 per call, took 0.3 ms of the
    // 0.42 ms pass over configuration 3's 31 M entries.)
    __device__ void flush(unsigned long long* bits_word, uint32_t rowptr_bit, uint32_t col_bit,
                          unsigned long long* diff_word) {
        __shared__ uint32_t block_bits[kBlock / kWave];
        __shared__ int64_t block_diff[kBlock / kWave];
        const uint32_t bits = wave_or((bad_rowptr ? rowptr_bit : 0u) | (bad_col ? col_bit : 0u));
        const int64_t d = wave_sum(desc - start_desc);
        if (__lane_id() == 0) {
            block_bits[threadIdx.x / kWave] = bits;
            block_diff[threadIdx.x / kWave] = d;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t b = 0;
            int64_t t = 0;
            for (int i = 0; i < kBlock / kWave; ++i) {
                b |= block_bits[i];
                t += block_diff[i];
            }
            if (b) atomicOr(bits_word, static_cast<unsigned long long>(b));
            if (t) atomicAdd(diff_word, static_cast<unsigned long long>(t));
        }
    }
};

// Record of node v as the walks read it: {v, row begin, degree, 0}, with
// degree kRecBadNode for an id outside [0, num_nodes) and kRecBadRow for a
// row outside [0, num_edges] or decreasing.
__device__ __forceinline__ int4 node_record(const int64_t* __restrict__ rowptr, int64_t v,
                                            int64_t num_nodes, int64_t num_edges) {
    int4 r = make_int4(static_cast<int32_t>(v), 0, kRecBadNode, 0);
    if (node_ok(v, num_nodes)) {
        const RowBounds rb = load_row(rowptr, v);
        if (row_ok(rb, num_edges)) {
            r.y = static_cast<int32_t>(rb.begin);
            r.z = static_cast<int32_t>(rb.end - rb.begin);
        } else {
            r.z = kRecBadRow;
        }
    }
    return r;
}

// The same record from the int32 row starts row32 (row32[v] = rowptr[v], or
// -1 for an entry outside [0, num_edges]; see row32_kernel): the row is
// valid iff row32[v] >= 0 and row32[v + 1] >= row32[v], as row_ok decides on
// rowptr.  The table is half the size of rowptr, so twice as much of it stays
// in each XCD's L2 while a preparation pass gathers rows for every entry.
__device__ __forceinline__ int4 node_record32(const int32_t* __restrict__ row32, int64_t v,
                                              int64_t num_nodes) {
    typedef int32_t i32x2 __attribute__((ext_vector_type(2), aligned(4)));
    int4 r = make_int4(static_cast<int32_t>(v), 0, kRecBadNode, 0);
    if (node_ok(v, num_nodes)) {
        const i32x2 b = *reinterpret_cast<const i32x2*>(row32 + v);
        if (b.x >= 0 && b.y >= b.x) {
            r.y = b.x;
            r.z = b.y - b.x;
        } else {
            r.z = kRecBadRow;
        }
    }
    return r;
}

// row32[v] = rowptr[v] as int32 for v in [0, num_nodes], -1 for an entry
// outside [0, num_edges] (num_edges < 2^31).
__global__ __launch_bounds__(kBlock) void row32_kernel(const int64_t* __restrict__ rowptr,
                                                       int64_t num_nodes, int64_t num_edges,
                                                       int32_t* __restrict__ row32) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t v = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; v <= num_nodes;
         v += stride) {
        const int64_t x = rowptr[v];
        row32[v] = x >= 0 && x <= num_edges ? static_cast<int32_t>(x) : -1;
    }
}

// Hub slot of a node record for the node2vec record walk: the slot of its
// bitmap when its row has one (degree at or above the threshold h), else -1.
__device__ __forceinline__ int4 with_slot(int4 r, const HubBitmaps& hubs, int64_t h) {
    r.w = r.z >= 0 && r.z >= h ? hubs.slot_of[r.x] : -1;
    return r;
}

// Edge records (see EdgeRecord); optionally (index.count > 0) also the
// levels of the node2vec walk's search index: col as int32 and its samples
// col32[16^k * i].  With rec == nullptr (the node2vec walk's CSR mode) only
// the index is written, with -1 for a col value outside [0, num_nodes), and
// no rowptr is read.  With a non-null work pointer the same pass validates the
// whole CSR (status bits into work[0]) and counts into work[2] the row
// descents that start no row (work[3] stays 0): the node2vec walk takes its
// rows as sorted when work[2] == work[3].  With hubs.max > 0 every record's pad word holds its node's
// hub slot (hub_assign_kernel ran before), else -1.  With a non-null row32
// (row32_kernel ran before) the rows are gathered from it instead of rowptr.
__global__ __launch_bounds__(kBlock) void edge_record_kernel(const int64_t* __restrict__ rowptr,
                                                             const int64_t* __restrict__ col,
                                                             int64_t num_nodes, int64_t num_edges,
                                                             EdgeRecord* __restrict__ rec,
                                                             IndexLevels index, StartRecords starts,
                                                             int64_t* work, HubBitmaps hubs,
                                                             const int32_t* __restrict__ row32) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t h = hubs.max > 0 ? hubs.info[0] : INT64_MAX;
    CsrCheck check;
    for (int64_t e = gid; e < num_edges; e += stride) {
        const int64_t c = col[e];
        if (work) check.edge(col, num_nodes, e, c);
        i32x4 r = {static_cast<int32_t>(c), 0, kRecBadNode, 0};
        if (!rec) {
            if (!node_ok(c, num_nodes)) r.x = -1;
        } else {
            if (row32) {
                const int4 n4 = node_record32(row32, c, num_nodes);
                r.y = n4.y;
                r.z = n4.z;
            } else if (node_ok(c, num_nodes)) {
                const RowBounds rb = load_row(rowptr, c);
                if (row_ok(rb, num_edges)) {
                    r.y = static_cast<int32_t>(rb.begin);
                    r.z = static_cast<int32_t>(rb.end - rb.begin);
                } else {
                    r.z = kRecBadRow;
                }
            }
            r.w = r.z >= 0 && r.z >= h ? hubs.slot_of[c] : -1;
            *reinterpret_cast<i32x4*>(rec + e) = r;
        }
        if (index.count > 0) {
            index.level[0][e] = r.x;
            // e is a multiple of 16^k for k = 1 .. while its low 4k bits are 0
            for (int k = 1; k < index.count && (e & ((int64_t{1} << (4 * k)) - 1)) == 0; ++k)
                index.level[k][e >> (4 * k)] = r.x;
        }
    }
    for (int64_t n = gid; n < starts.num_walks; n += stride)
        *reinterpret_cast<int4*>(starts.init + n) =
            with_slot(row32 ? node_record32(row32, starts.start[n], num_nodes)
                            : node_record(rowptr, starts.start[n], num_nodes, num_edges),
                      hubs, h);
    if (work) {
        check.nodes(rowptr, num_nodes, col, num_edges, gid, stride);
        unsigned long long* w = reinterpret_cast<unsigned long long*>(work);
        check.flush(w, MLXC_STATUS_BAD_ROW, MLXC_STATUS_BAD_NODE, w + 2);
    }
}

// Rows per degree class into info[2 + k] (k = floor(log2(deg)) - kHubMinLog,
// the last class holding every larger degree): per-block counts in LDS, one
// atomic per class per block.  info must start at zero.
__global__ __launch_bounds__(kBlock) void hub_count_kernel(const int64_t* __restrict__ rowptr,
                                                           int64_t num_nodes, int64_t num_edges,
                                                           int64_t* info) {
    __shared__ int32_t cnt[kHubDegreeClasses];
    if (threadIdx.x < kHubDegreeClasses) cnt[threadIdx.x] = 0;
    __syncthreads();
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t u = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; u < num_nodes;
         u += stride) {
        const RowBounds rb = load_row(rowptr, u);
        const int64_t d = rb.end - rb.begin;
        if (!row_ok(rb, num_edges) || d < kHubMinDegree) continue;
        const int k = min(63 - __clzll(static_cast<unsigned long long>(d)) - kHubMinLog,
                          kHubDegreeClasses - 1);
        atomicAdd(&cnt[k], 1);
    }
    __syncthreads();
    if (threadIdx.x < kHubDegreeClasses && cnt[threadIdx.x] > 0)
        atomicAdd(reinterpret_cast<unsigned long long*>(info + 2 + threadIdx.x),
                  static_cast<unsigned long long>(cnt[threadIdx.x]));
}

// The smallest degree threshold 2^(kHubMinLog + k), at least min_degree,
// whose rows fit max slots (INT64_MAX when none does).
__device__ __forceinline__ int64_t hub_threshold(const int64_t* info, int32_t max,
                                                 int64_t min_degree) {
    int64_t above = 0, h = INT64_MAX;
    for (int k = kHubDegreeClasses - 1; k >= 0; --k) {
        const int64_t hk = int64_t{1} << (kHubMinLog + k);
        above += info[2 + k];
        if (above > max || hk < min_degree) break;
        h = hk;
    }
    return h;
}

// info[0] = the threshold; every row at or above it gets the next slot
// (info[1] counts them; the order of slots is immaterial).
__global__ __launch_bounds__(kBlock) void hub_assign_kernel(const int64_t* __restrict__ rowptr,
                                                            int64_t num_nodes, int64_t num_edges,
                                                            HubBitmaps hubs, int64_t min_degree) {
    const int64_t h = hub_threshold(hubs.info, hubs.max, min_degree);
    if (blockIdx.x == 0 && threadIdx.x == 0) hubs.info[0] = h;
    if (h == INT64_MAX) return;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t u = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; u < num_nodes;
         u += stride) {
        const RowBounds rb = load_row(rowptr, u);
        if (!row_ok(rb, num_edges) || rb.end - rb.begin < h) continue;
        const int64_t slot = static_cast<int64_t>(
            atomicAdd(reinterpret_cast<unsigned long long*>(hubs.info + 1), 1ull));
        hubs.slot_of[u] = static_cast<int32_t>(slot);  // slot < max: the threshold ensures it
        hubs.node_of[slot] = static_cast<int32_t>(u);
    }
}

// Builds the bitmaps of the assigned slots, each in chunks of
// kHubChunkWords words: a block clears its chunk in LDS, sets the bits of the
// row's entries that fall in it (LDS atomics), then stores the chunk whole,
// so no separate clearing pass and no global atomics are needed.  On sorted
// rows (rows == MLXC_ROWS_SORTED, or DETECT with work[2] == work[3] from the
// preparation pass, which must have run) each chunk binary-searches the
// range of entries it holds; otherwise it scans the whole row.  Entries
// outside [0, num_nodes) are left out (the preparation pass reports them).
constexpr int kHubChunkWords = 8192;  // 32 KB of LDS: 2^18 nodes per chunk
constexpr int64_t kHubScanEntries = 16 * kBlock;  // rows up to this are scanned by every chunk
constexpr int kHubLoads = 8;

// lower_bound of v in the sorted a[lo, hi), by the whole block: each round
// every thread compares one of kBlock evenly spaced samples, and the count of
// samples below v (a block-wide reduction) narrows the range kBlock-fold, so
// a row of d entries takes about log256(d) + 1 dependent reads instead of
// log2(d).  Every thread of the block must call it; all get the same result.
__device__ int64_t block_lower_bound(const int64_t* __restrict__ a, int64_t lo, int64_t hi,
                                     int64_t v) {
    while (hi - lo > kBlock) {
        const int64_t step = (hi - lo + kBlock - 1) / kBlock;
        const int64_t k = threadIdx.x;  // sample k sits at lo + k * step
        const int64_t at = lo + k * step;
        const int c = __syncthreads_count(at < hi && a[at] < v);
        // samples 0 .. c-1 are below v and sample c (if any) is not
        const int64_t new_lo = c == 0 ? lo : lo + (c - 1) * step + 1;
        const int64_t new_hi = lo + c * step < hi ? lo + c * step : hi;
        lo = new_lo;
        hi = new_hi;
    }
    const int64_t at = lo + threadIdx.x;
    return lo + __syncthreads_count(at < hi && a[at] < v);
}

__global__ __launch_bounds__(kBlock) void hub_build_kernel(const int64_t* __restrict__ rowptr,
                                                           const int64_t* __restrict__ col,
                                                           int64_t num_nodes, HubBitmaps hubs,
                                                           int32_t rows, const int64_t* work) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __shared__ uint32_t lw[kHubChunkWords];
    const bool sorted = rows == MLXC_ROWS_SORTED || (rows == MLXC_ROWS_DETECT && work[2] == work[3]);
    const int64_t chunks = (hubs.words + kHubChunkWords - 1) / kHubChunkWords;
    const int64_t units = hubs.info[1] * chunks;
    for (int64_t unit = blockIdx.x; unit < units; unit += gridDim.x) {
        const int64_t slot = unit / chunks, chunk = unit % chunks;
        const int64_t w0 = chunk * kHubChunkWords;  // first word of the chunk
        const int64_t nw = min(static_cast<int64_t>(kHubChunkWords), hubs.words - w0);
        for (int i = threadIdx.x; i < nw; i += kBlock) lw[i] = 0u;
        __syncthreads();
        const RowBounds rb = load_row(rowptr, hubs.node_of[slot]);  // a valid row (assigned)
        int64_t first = rb.begin, last = rb.end;
        if (sorted && chunks > 1 && rb.end - rb.begin > kHubScanEntries) {
            // the entries in [32 w0, 32 (w0 + nw)); shorter rows are scanned whole
            first = block_lower_bound(col, rb.begin, rb.end, 32 * w0);
            last = block_lower_bound(col, first, rb.end, 32 * (w0 + nw));
        }
        // kHubLoads loads per thread issued before any is used (indices past
        // the range clamped to its last entry), one memory round trip each
        for (int64_t i0 = first + threadIdx.x; i0 < last; i0 += kHubLoads * kBlock) {
            int64_t c[kHubLoads];
#pragma unroll
            for (int u = 0; u < kHubLoads; ++u) {
                const int64_t i = i0 + u * kBlock;
                c[u] = col[i < last ? i : last - 1];
            }
#pragma unroll
            for (int u = 0; u < kHubLoads; ++u) {
                const int64_t wi = (c[u] >> 5) - w0;
                if (i0 + u * kBlock < last && node_ok(c[u], num_nodes) && wi >= 0 && wi < nw)
                    atomicOr(&lw[wi], 1u << (c[u] & 31));
            }
        }
        __syncthreads();
        u32x4* out = reinterpret_cast<u32x4*>(hubs.bits + slot * hubs.words + w0);
        for (int64_t q = threadIdx.x; 4 * q < nw; q += kBlock)  // nw is a multiple of 4
            out[q] = u32x4{lw[4 * q], lw[4 * q + 1], lw[4 * q + 2], lw[4 * q + 3]};
        __syncthreads();
    }
}

// Row hash tables (see row_hashed in walk_device.h), built in LDS by one
// wavefront per table and stored whole with 16-byte stores: clear the table,
// insert the row's entries (col32; -1, a malformed id, is left out) with an
// LDS counter per bucket, moving on to the next bucket of the row when one is
// full, store.  A table holds fewer than 2 entries per 16 slots of capacity
// (or its whole row in one bucket), so an insertion always finds a bucket.
//
// Two launches.  hash_short_kernel: each wavefront reads the row starts of
// groups of 64 consecutive rows, builds the tables of the short rows (at most
// 64 entries) kHashBatch at a time, their entry loads issued together so that
// one memory round trip serves the batch, and appends the long rows to a list
// (one atomic per group).  hash_long_kernel: the wavefronts take the listed
// rows round robin, one row at a time with all of its loads issued first.
// The list spreads the long rows evenly: they crowd together where degrees
// are skewed (R-MAT gives low ids, and ids of few set bits, high degrees),
// and handed out by row id a few wavefronts got most of them
// (configuration 3: 71 long rows on one wavefront against 6.6 on average,
// 0.47 ms for the long rows).  Each launch gives its waves only the LDS its
// rows need.  hub_info: rows of at least the hub threshold info[0] have
// bitmaps and no table (null: no bitmaps in this call).
constexpr int kHashTableMax = ((kHashMaxDegree - 1) >> 3) + 1;  // buckets of the longest table
constexpr int kHashBatch = 8;
constexpr int kHashShortMax = kWave;                            // entries of a short row
constexpr int kHashShortBuckets = (kHashShortMax >> 3) + 1;     // buckets of its table

// Inserts c (>= 0) into the table of nb buckets at sl / fl (wave-local LDS).
__device__ __forceinline__ void hash_insert(int32_t* sl, int32_t* fl, int32_t nb, int32_t c) {
    int32_t bk = hash_bucket(c, nb);
    while (true) {
        const int32_t at = atomicAdd(&fl[bk], 1);
        if (at < kSearchBlock) {
            sl[bk * kSearchBlock + at] = c;
            return;
        }
        bk = bk + 1 == nb ? 0 : bk + 1;
    }
}

// Stores the table of nb buckets at sl to its region (all lanes).
__device__ __forceinline__ void hash_store(int32_t* __restrict__ table, const int32_t* sl,
                                           int32_t nb, int32_t begin, int32_t node, int lane) {
    int4* out = reinterpret_cast<int4*>(table + hash_region(begin, node) * kSearchBlock);
    for (int q = lane; q < nb * (kSearchBlock / 4); q += kWave)
        out[q] = make_int4(sl[4 * q], sl[4 * q + 1], sl[4 * q + 2], sl[4 * q + 3]);
}

__global__ __launch_bounds__(kBlock) void hash_short_kernel(const int32_t* __restrict__ row32,
                                                            const int32_t* __restrict__ col32,
                                                            int64_t num_nodes,
                                                            const int64_t* __restrict__ hub_info,
                                                            int32_t* __restrict__ table,
                                                            int32_t* __restrict__ long_rows,
                                                            unsigned long long* long_count) {
    constexpr int kWaves = kBlock / kWave;
    constexpr int kArea = kHashBatch * kHashShortBuckets;  // buckets of a wave's batch
    constexpr int kPend = 2 * kWave;  // long rows a wave lists before appending them
    __shared__ int32_t slots[kWaves][kArea * kSearchBlock];
    __shared__ int32_t fill[kWaves][kArea];
    __shared__ int32_t pend[kWaves][kPend];
    const int w = threadIdx.x / kWave;
    const int lane = static_cast<int>(__lane_id());
    const int64_t h = hub_info ? hub_info[0] : INT64_MAX;
    int32_t* const sl = slots[w];
    int32_t* const fl = fill[w];
    int32_t* const pl = pend[w];
    int npend = 0;  // wave-uniform
    // the listed long rows go to the list with one atomic per flush, not one
    // per group (whose return each group would otherwise wait for)
    auto flush = [&]() {
        uint32_t at = 0;
        if (lane == 0)
            at = static_cast<uint32_t>(atomicAdd(long_count, static_cast<unsigned long long>(npend)));
        at = __builtin_amdgcn_readlane(at, 0);
        for (int k = lane; k < npend; k += kWave) long_rows[at + k] = pl[k];
        npend = 0;
        wave_sync();
    };
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * kWaves + w; g * kWave < num_nodes;
         g += waves) {
        const int64_t base = g * kWave;
        const int64_t u = base + lane;
        int32_t b = 0, d = 0;
        bool mine = false;
        if (u < num_nodes) {
            const int32_t rb = row32[u], re = row32[u + 1];
            if (rb >= 0 && re >= rb) {
                b = rb;
                d = re - rb;
                mine = row_hashed(rb, d, h);
            }
        }
        const bool is_long = mine && d > kHashShortMax;
        const uint64_t longs = __ballot(is_long);
        if (longs) {  // list the group's long rows (at most num_nodes in all)
            if (npend + __popcll(longs) > kPend) flush();
            if (is_long) pl[npend + lane_rank(longs)] = static_cast<int32_t>(u);
            npend += __popcll(longs);
            wave_sync();
        }
        uint64_t shorts = __ballot(mine && !is_long);
        while (shorts) {  // wave-uniform
            int32_t rb[kHashBatch], rd[kHashBatch], node[kHashBatch], v[kHashBatch];
#pragma unroll
            for (int j = 0; j < kHashBatch; ++j) {
                rb[j] = 0;
                rd[j] = 0;
                node[j] = 0;
                if (shorts) {
                    const int src = __builtin_ctzll(shorts);
                    shorts &= shorts - 1;
                    rb[j] = __builtin_amdgcn_readlane(b, src);
                    rd[j] = __builtin_amdgcn_readlane(d, src);
                    node[j] = static_cast<int32_t>(base + src);
                }
                // unconditional (the index clamped into the row, or entry 0
                // for an unused batch place), so the loads are in flight together
                v[j] = col32[rb[j] + min(lane, max(rd[j] - 1, 0))];
            }
#pragma unroll
            for (int j = 0; j < kHashBatch; ++j) {
                const int32_t nb = rd[j] > 0 ? hash_buckets(rd[j]) : 0;
                int32_t* const tj = sl + j * kHashShortBuckets * kSearchBlock;
                for (int i = lane; i < nb * kSearchBlock; i += kWave) tj[i] = -1;
                if (lane < nb) fl[j * kHashShortBuckets + lane] = 0;
            }
            wave_sync();
#pragma unroll
            for (int j = 0; j < kHashBatch; ++j)
                if (lane < rd[j] && v[j] >= 0)
                    hash_insert(sl + j * kHashShortBuckets * kSearchBlock, fl + j * kHashShortBuckets,
                                hash_buckets(rd[j]), v[j]);
            wave_sync();
#pragma unroll
            for (int j = 0; j < kHashBatch; ++j)
                if (rd[j] > 0)
                    hash_store(table, sl + j * kHashShortBuckets * kSearchBlock,
                               hash_buckets(rd[j]), rb[j], node[j], lane);
            wave_sync();
        }
    }
    if (npend > 0) flush();
}

__global__ __launch_bounds__(kBlock) void hash_long_kernel(const int32_t* __restrict__ row32,
                                                           const int32_t* __restrict__ col32,
                                                           int32_t* __restrict__ table,
                                                           const int32_t* __restrict__ long_rows,
                                                           const unsigned long long* long_count) {
    constexpr int kWaves = kBlock / kWave;
    __shared__ int32_t slots[kWaves][kHashTableMax * kSearchBlock];
    __shared__ int32_t fill[kWaves][kHashTableMax];
    const int w = threadIdx.x / kWave;
    const int lane = static_cast<int>(__lane_id());
    int32_t* const sl = slots[w];
    int32_t* const fl = fill[w];
    const int64_t n = static_cast<int64_t>(*long_count);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + w; i < n; i += waves) {
        const int32_t u = long_rows[i];
        const int32_t rb = row32[u], rd = row32[u + 1] - rb;  // a listed row: valid, 65..1023
        const int32_t nb = hash_buckets(rd);
        // every round's load first (indices clamped into the row), then the
        // inserts: a load behind an insert would wait for it
        constexpr int kRounds = (kHashMaxDegree + kWave - 1) / kWave;
        const int rounds = (rd + kWave - 1) / kWave;
        int32_t v[kRounds];
#pragma unroll
        for (int r = 0; r < kRounds; ++r)
            if (r < rounds) v[r] = col32[rb + min(lane + r * kWave, rd - 1)];
        for (int k = lane; k < nb * kSearchBlock; k += kWave) sl[k] = -1;
        for (int k = lane; k < nb; k += kWave) fl[k] = 0;
        wave_sync();
#pragma unroll
        for (int r = 0; r < kRounds; ++r)
            if (r < rounds && lane + r * kWave < rd && v[r] >= 0) hash_insert(sl, fl, nb, v[r]);
        wave_sync();
        hash_store(table, sl, nb, rb, u, lane);
        wave_sync();
    }
}

int launch_hash_build(const int32_t* row32, const int32_t* col32, int64_t num_nodes,
                      const int64_t* hub_info, int32_t* table, int32_t* long_rows,
                      int64_t* long_count, hipStream_t stream) {
    if (num_nodes <= 0) return MLXC_OK;
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    const int64_t groups = (num_nodes + kWave - 1) / kWave;  // one per wavefront and round
    const int64_t want = (groups + kBlock / kWave - 1) / (kBlock / kWave);
    const int64_t cap = static_cast<int64_t>(info.cus) * 8;
    const int grid = static_cast<int>(want < cap ? want : cap);
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kWave), 0, stream, long_count, 1);
    hipLaunchKernelGGL(hash_short_kernel, dim3(grid), dim3(kBlock), 0, stream, row32, col32,
                       num_nodes, hub_info, table, long_rows,
                       reinterpret_cast<unsigned long long*>(long_count));
    hipLaunchKernelGGL(hash_long_kernel, dim3(static_cast<int>(cap)), dim3(kBlock), 0, stream,
                       row32, col32, table, long_rows,
                       reinterpret_cast<const unsigned long long*>(long_count));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

// The search index alone (the node2vec walk's CSR mode: no records, no rowptr
// read per edge): col32 = col with -1 for a value outside [0, num_nodes),
// plus its samples col32[16^k * i]; with a non-null work pointer the same
// pass validates the CSR, as edge_record_kernel does.  Each thread takes four
// consecutive entries per iteration (two 16-byte loads, one 16-byte store);
// col must be 16-byte aligned.
__global__ __launch_bounds__(kBlock) void edge_index_kernel(const int64_t* __restrict__ rowptr,
                                                            const int64_t* __restrict__ col,
                                                            int64_t num_nodes, int64_t num_edges,
                                                            IndexLevels index, StartRecords starts,
                                                            int64_t* work) {
    typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    CsrCheck check;
    for (int64_t q = gid; 4 * q < num_edges; q += stride) {
        const int64_t e0 = 4 * q;
        int64_t c[4];
        if (e0 + 4 <= num_edges) {
            const i64x2 a = reinterpret_cast<const i64x2*>(col + e0)[0];
            const i64x2 b = reinterpret_cast<const i64x2*>(col + e0)[1];
            c[0] = a.x; c[1] = a.y; c[2] = b.x; c[3] = b.y;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = e0 + k < num_edges ? col[e0 + k] : 0;
        }
        int32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t e = e0 + k;
            v[k] = node_ok(c[k], num_nodes) ? static_cast<int32_t>(c[k]) : -1;
            if (work && e < num_edges) {
                if (!node_ok(c[k], num_nodes)) check.bad_col = true;
                if (e >= 1 && c[k] < (k ? c[k - 1] : col[e - 1])) ++check.desc;
            }
        }
        // col32 is padded to whole 16-entry blocks, so the last store fits
        *reinterpret_cast<i32x4*>(index.level[0] + e0) = i32x4{v[0], v[1], v[2], v[3]};
        if ((e0 & 15) == 0) {
            for (int k = 1; k < index.count && (e0 & ((int64_t{1} << (4 * k)) - 1)) == 0; ++k)
                index.level[k][e0 >> (4 * k)] = v[0];
        }
    }
    for (int64_t n = gid; n < starts.num_walks; n += stride)
        *reinterpret_cast<int4*>(starts.init + n) =
            node_record(rowptr, starts.start[n], num_nodes, num_edges);
    if (work) {
        check.nodes(rowptr, num_nodes, col, num_edges, gid, stride);
        unsigned long long* w = reinterpret_cast<unsigned long long*>(work);
        check.flush(w, MLXC_STATUS_BAD_ROW, MLXC_STATUS_BAD_NODE, w + 2);
    }
}

// The uniform record walk's whole preparation in one launch (a small call
// is bound by launch latency): the call's status words zeroed, the edge
// record of every CSR entry, then the start record of every walk, as
// EdgeRecord or (kPacked) in the 8-byte format fmt.  The start records
// follow the edge records: init = recs + num_edges.
template <bool kPacked>
__global__ __launch_bounds__(kBlock) void record_prep_kernel(const int64_t* __restrict__ rowptr,
                                                             const int64_t* __restrict__ col,
                                                             const int64_t* __restrict__ start,
                                                             int64_t num_nodes, int64_t num_edges,
                                                             int64_t num_walks,
                                                             void* __restrict__ recs,
                                                             PackedFormat fmt,
                                                             int64_t* __restrict__ work) {
    if (blockIdx.x == 0 && threadIdx.x < MLXC_WORK_WORDS) work[threadIdx.x] = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
         i < num_edges + num_walks; i += stride) {
        const int4 r = node_record(rowptr, i < num_edges ? col[i] : start[i - num_edges],
                                   num_nodes, num_edges);
        if (kPacked)
            static_cast<uint64_t*>(recs)[i] = fmt.pack(r.x, r.y, r.z);
        else
            static_cast<int4*>(recs)[i] = r;
    }
}

// Start records: walk n's start node in the edge-record format, so a slot
// beginning a walk and a slot taking a step both issue the same single 16-byte
// read.  Written by walk_init_kernel (one coalesced pass over start).
__global__ __launch_bounds__(kBlock) void walk_init_kernel(const int64_t* __restrict__ rowptr,
                                                           const int64_t* __restrict__ start,
                                                           int64_t num_nodes, int64_t num_edges,
                                                           int64_t num_walks,
                                                           EdgeRecord* __restrict__ init,
                                                           int64_t* __restrict__ work) {
    if (blockIdx.x == 0 && threadIdx.x < MLXC_WORK_WORDS) work[threadIdx.x] = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; n < num_walks;
         n += stride)
        *reinterpret_cast<int4*>(init + n) = node_record(rowptr, start[n], num_nodes, num_edges);
}

// work[0] |= MLXC_CSR_BAD_ROWPTR / MLXC_CSR_BAD_COL bits; work[1] counts the
// positions i >= 1 with col[i] < col[i-1] that start no non-empty row (work[2]
// stays 0).  Rows are sorted iff work[1] == work[2].
__global__ __launch_bounds__(kBlock) void csr_check_kernel(const int64_t* __restrict__ rowptr,
                                                           int64_t V,
                                                           const int64_t* __restrict__ col,
                                                           int64_t E, int64_t* work) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    CsrCheck check;
    check.nodes(rowptr, V, col, E, gid, stride);
    for (int64_t i = gid; i < E; i += stride) check.edge(col, V, i, col[i]);
    unsigned long long* w = reinterpret_cast<unsigned long long*>(work);
    check.flush(w, MLXC_CSR_BAD_ROWPTR, MLXC_CSR_BAD_COL, w + 1);
}

// After csr_check_kernel, on a well-formed graph whose rows are all sorted:
// work[3] = 1 if some entry (u, v) has no entry (v, u).  Each thread takes
// runs of 16 consecutive entries; the run's row comes from a binary search of
// rowptr, then each entry's reverse from a binary search of row(v).
__global__ __launch_bounds__(kBlock) void csr_symmetry_kernel(const int64_t* __restrict__ rowptr,
                                                              int64_t V,
                                                              const int64_t* __restrict__ col,
                                                              int64_t E, int64_t* work) {
    constexpr int kRun = 16;
    if ((work[0] & (MLXC_CSR_BAD_ROWPTR | MLXC_CSR_BAD_COL)) || work[1] != work[2]) return;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    bool asym = false;
    for (int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * kRun; e0 < E;
         e0 += stride * kRun) {
        int64_t lo = 0, hi = V - 1;  // the last row u with rowptr[u] <= e0
        while (lo < hi) {
            const int64_t mid = hi - (hi - lo) / 2;
            if (rowptr[mid] <= e0) lo = mid;
            else hi = mid - 1;
        }
        int64_t u = lo;
        const int64_t e1 = e0 + kRun < E ? e0 + kRun : E;
        for (int64_t e = e0; e < e1; ++e) {
            while (rowptr[u + 1] <= e) ++u;  // (rowptr[V] = E > e ends it)
            const int64_t v = col[e];
            int64_t b = rowptr[v], n = rowptr[v + 1] - b;
            while (n > 0) {  // lower_bound of u in row(v)
                const int64_t half = n >> 1;
                if (col[b + half] < u) {
                    b += half + 1;
                    n -= half + 1;
                } else {
                    n = half;
                }
            }
            asym |= !(b < rowptr[v + 1] && col[b] == u);
        }
    }
    if (__any(asym) && __lane_id() == 0)
        atomicOr(reinterpret_cast<unsigned long long*>(work + 3), 1ull);
}

// The words csr_check_kernel left, turned into a walk's: work[0] = the
// MLXC_STATUS_* bits of the whole-graph check, work[1] = 0 (the walk queue),
// work[2] = 1 when every row is sorted (else 0), work[3] = 0.
__global__ void csr_status_kernel(int64_t* work) {
    if (threadIdx.x != 0) return;
    const int64_t bits = work[0];
    const bool sorted = work[1] == work[2];
    work[0] = ((bits & MLXC_CSR_BAD_ROWPTR) ? MLXC_STATUS_BAD_ROW : 0) |
              ((bits & MLXC_CSR_BAD_COL) ? MLXC_STATUS_BAD_NODE : 0);
    work[1] = 0;
    work[2] = sorted ? 1 : 0;
    work[3] = 0;
}

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

// ------------------------------------------------------------- launchers

int stream_grid(int64_t items, int blocks_per_cu, int& grid) {
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    int64_t g = (items + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(info.cus) * blocks_per_cu;
    if (g > cap) g = cap;
    grid = static_cast<int>(g < 1 ? 1 : g);
    return MLXC_OK;
}

int launch_zero_work(int64_t* d_work, hipStream_t stream) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kWave), 0, stream, d_work, MLXC_WORK_WORDS);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_edge_records(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                        int64_t num_edges, EdgeRecord* recs, const IndexLevels& index,
                        const StartRecords& starts, int64_t* check_work, hipStream_t stream,
                        const HubBitmaps& hubs, int32_t* row32) {
    int grid = 0;
    if (row32) {
        if (int rc = stream_grid(num_nodes + 1, 8, grid)) return rc;
        hipLaunchKernelGGL(row32_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                           num_edges, row32);
    }
    if (num_edges == 0 && !check_work && starts.num_walks == 0) return MLXC_OK;
    int64_t items = check_work && num_nodes > num_edges ? num_nodes : num_edges;
    if (starts.num_walks > items) items = starts.num_walks;
    if (int rc = stream_grid(items, 16, grid)) return rc;
    hipLaunchKernelGGL(edge_record_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, col,
                       num_nodes, num_edges, recs, index, starts, check_work, hubs,
                       static_cast<const int32_t*>(row32));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_hub_bitmaps(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                       int64_t num_edges, const HubBitmaps& hubs, int64_t min_degree,
                       hipStream_t stream) {
    if (hubs.max <= 0) return MLXC_OK;
    static_assert(kHubInfoWords <= kWave, "one zeroing thread per info word");
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kWave), 0, stream, hubs.info, kHubInfoWords);
    int grid = 0;
    if (int rc = stream_grid(num_nodes, 8, grid)) return rc;
    hipLaunchKernelGGL(hub_count_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                       num_edges, hubs.info);
    hipLaunchKernelGGL(hub_assign_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                       num_edges, hubs, min_degree);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_hub_build(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                     const HubBitmaps& hubs, int32_t rows, const int64_t* work,
                     hipStream_t stream) {
    if (hubs.max <= 0) return MLXC_OK;
    const int64_t chunks = (hubs.words + kHubChunkWords - 1) / kHubChunkWords;
    int grid = 0;  // four 32 KB blocks per CU
    if (int rc = stream_grid(static_cast<int64_t>(hubs.max) * chunks * kBlock, 4, grid)) return rc;
    hipLaunchKernelGGL(hub_build_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, col,
                       num_nodes, hubs, rows, work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_edge_index(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                      int64_t num_edges, const IndexLevels& index, const StartRecords& starts,
                      int64_t* check_work, hipStream_t stream, int32_t* row32) {
    if (reinterpret_cast<uintptr_t>(col) % 16 != 0)  // the record pass reads any alignment
        return launch_edge_records(rowptr, col, num_nodes, num_edges, nullptr, index, starts,
                                   check_work, stream, HubBitmaps{}, row32);
    int grid = 0;
    if (row32) {
        if (int rc = stream_grid(num_nodes + 1, 8, grid)) return rc;
        hipLaunchKernelGGL(row32_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                           num_edges, row32);
    }
    if (num_edges == 0 && !check_work && starts.num_walks == 0) return MLXC_OK;
    const int64_t quads = (num_edges + 3) / 4;
    int64_t items = check_work && num_nodes > quads ? num_nodes : quads;
    if (starts.num_walks > items) items = starts.num_walks;
    if (int rc = stream_grid(items, 16, grid)) return rc;
    hipLaunchKernelGGL(edge_index_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, col,
                       num_nodes, num_edges, index, starts, check_work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_walk_init(const int64_t* rowptr, const int64_t* start, int64_t num_nodes,
                     int64_t num_edges, int64_t num_walks, EdgeRecord* init, int64_t* work,
                     hipStream_t stream) {
    int grid = 0;
    if (int rc = stream_grid(num_walks, 16, grid)) return rc;
    hipLaunchKernelGGL(walk_init_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, start,
                       num_nodes, num_edges, num_walks, init, work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_record_prep(const int64_t* rowptr, const int64_t* col, const int64_t* start,
                       int64_t num_nodes, int64_t num_edges, int64_t num_walks, void* recs,
                       const PackedFormat* packed, int64_t* work, hipStream_t stream) {
    int grid = 0;
    if (int rc = stream_grid(num_edges + num_walks, 16, grid)) return rc;
    if (packed)
        hipLaunchKernelGGL(record_prep_kernel<true>, dim3(grid), dim3(kBlock), 0, stream, rowptr,
                           col, start, num_nodes, num_edges, num_walks, recs, *packed, work);
    else
        hipLaunchKernelGGL(record_prep_kernel<false>, dim3(grid), dim3(kBlock), 0, stream, rowptr,
                           col, start, num_nodes, num_edges, num_walks, recs, PackedFormat{0, 0, 0},
                           work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_csr_check(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                     int64_t num_edges, int64_t* d_work, hipStream_t stream) {
    int grid = 0;
    if (int rc = stream_grid(num_nodes > num_edges ? num_nodes : num_edges, 8, grid)) return rc;
    hipLaunchKernelGGL(csr_check_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                       col, num_edges, d_work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_copy_word(const int64_t* d_src, int64_t* d_dst, hipStream_t stream) {
    hipLaunchKernelGGL(copy_word_kernel, dim3(1), dim3(kWave), 0, stream, d_src, d_dst);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_csr_symmetry(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                        int64_t num_edges, int64_t* d_work, hipStream_t stream) {
    if (num_edges == 0 || num_nodes == 0) return MLXC_OK;
    int grid = 0;
    if (int rc = stream_grid((num_edges + 15) / 16, 16, grid)) return rc;
    hipLaunchKernelGGL(csr_symmetry_kernel, dim3(grid), dim3(kBlock), 0, stream, rowptr, num_nodes,
                       col, num_edges, d_work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_csr_status(int64_t* d_work, hipStream_t stream) {
    hipLaunchKernelGGL(csr_status_kernel, dim3(1), dim3(kWave), 0, stream, d_work);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int launch_philox_fill(float* out, int64_t n, uint64_t seed, hipStream_t stream) {
    if (n == 0) return MLXC_OK;
    int grid = 0;
    if (int rc = stream_grid((n + 3) / 4, 16, grid)) return rc;
    hipLaunchKernelGGL(philox_fill_kernel, dim3(grid), dim3(kBlock), 0, stream, out, n,
                       static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

}  // namespace mlxc
