// CSR construction on the device: the step before the walk.  The reference
// tests build their CSR on the host (/root/reference/tests/
// test_random_walk.py:23-28: mlx_graphs 0.0.7 sort_edge_index, then rowptr
// from np.unique counts and a cumsum); this does the same on the GPU, with
// rowptr over all num_nodes rows.
//
// Method: an LSD radix sort of packed keys (row << cbits | col), cbits =
// bits(num_nodes - 1), sorting only the 2 * cbits bits that can be non-zero,
// 8 bits per pass.  Keys are stored in 4 bytes when they fit (num_nodes <=
// 65536), in 5 or 6 (a 32-bit and an 8- or 16-bit array) up to 40 or 48 bits,
// else in 8.  Each pass is three launches (four when rows of counts are long,
// below) and needs no inter-block waiting:
//   radix_hist_kernel     per 8192-key tile, a 256-digit histogram, written
//                         digit-major (hist[d * tiles + tile]);
//   row_scan_kernel       an exclusive scan of each digit's row of tile
//                         counts, one block per digit, and the digit totals
//                         (rows over kRowScanTiles tiles: a scan of the whole
//                         array, two launches, positions included);
//   radix_scatter_kernel  stable rank of each key inside its tile (wavefront
//                         match of the digit), reorder of the tile in LDS,
//                         then stores in digit runs; a (digit, tile)'s first
//                         output position is its row prefix plus the digit
//                         totals before it.
// Each scatter also writes every key's digit of the next pass into a byte
// array beside the keys, so that the next histogram reads 1 byte per key
// instead of the key.  The first pass reads the caller's (row, col) arrays
// directly (and the reversed pairs, for symmetrize); the last pass's keys go
// to csr_emit_kernel, which writes col, marks row starts and, with dedup,
// drops repeated keys.
// rowptr is filled with the entry count, row starts are written into it, and a
// reverse inclusive min-scan gives empty rows the start of the next row.
#include "walk_host.h"

namespace mlxc {

namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;  // 256 digits
constexpr int kItems = 16;               // keys (or values) per thread
constexpr int kChunk = kBlock * kItems;  // 4096 values per block of the scan and finish kernels
constexpr int kWaves = kBlock / kWave;

// Radix tiles: 512 threads x 16 keys.  8192 keys per tile give each digit a
// run of 32 keys (256 bytes of 64-bit keys) on average in the scatter, which
// keeps its stores in whole lines; two blocks fit a CU's LDS.
#ifndef MLXC_CSR_SORT_THREADS
#define MLXC_CSR_SORT_THREADS 512
#endif
constexpr int kSortThreads = MLXC_CSR_SORT_THREADS;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSortTile = kSortThreads * kItems;
constexpr int kWaveTile = kWave * kItems;

static_assert(kRadix == kBlock && kSortThreads >= kRadix, "one digit per thread");

constexpr int kOpSum = 0;
constexpr int kOpMin = 1;

struct EdgeSrc {
    const int64_t* row;
    const int64_t* col;
    int64_t num_edges;  // entries of row / col (the list before symmetrizing)
    int64_t num_nodes;
    int cbits;          // bits of the col field of a key
};

// Key arrays.  Keys of up to 32 bits are stored whole; keys of 33 to 40 (48)
// bits as a 32-bit array of their low halves and an 8-bit (16-bit) array of
// their high bits, 5 (6) bytes a key instead of 8, so every pass over them
// moves that many fewer bytes; wider keys as 64-bit words.  A store is a set
// of device pointers passed by value; K is the key's type in registers.
struct Keys32 {
    using K = uint32_t;
    uint32_t* p;
    __device__ __forceinline__ K load(int64_t i) const { return p[i]; }
    __device__ __forceinline__ void store(int64_t i, K k) const { p[i] = k; }
};
struct Keys40 {
    using K = uint64_t;
    uint32_t* lo;
    uint8_t* hi;
    __device__ __forceinline__ K load(int64_t i) const {
        return (static_cast<uint64_t>(hi[i]) << 32) | lo[i];
    }
    __device__ __forceinline__ void store(int64_t i, K k) const {
        lo[i] = static_cast<uint32_t>(k);
        hi[i] = static_cast<uint8_t>(k >> 32);
    }
};
struct Keys48 {
    using K = uint64_t;
    uint32_t* lo;
    uint16_t* hi;
    __device__ __forceinline__ K load(int64_t i) const {
        return (static_cast<uint64_t>(hi[i]) << 32) | lo[i];
    }
    __device__ __forceinline__ void store(int64_t i, K k) const {
        lo[i] = static_cast<uint32_t>(k);
        hi[i] = static_cast<uint16_t>(k >> 32);
    }
};
struct Keys64 {
    using K = uint64_t;
    uint64_t* p;
    __device__ __forceinline__ K load(int64_t i) const { return p[i]; }
    __device__ __forceinline__ void store(int64_t i, K k) const { p[i] = k; }
};

// An id outside [0, num_nodes) sets `bad` and becomes 0 (each id on its own),
// so that every index derived from a key stays in bounds.
__device__ __forceinline__ int64_t clamp_id(int64_t v, int64_t num_nodes, bool& bad) {
    const bool ok = static_cast<uint64_t>(v) < static_cast<uint64_t>(num_nodes);
    bad |= !ok;
    return ok ? v : 0;
}

// Addresses of entry i's row and col ids (i >= num_edges: the reversed pair
// of entry i - num_edges), chosen by a select rather than a branch.
__device__ __forceinline__ const int64_t* src_row_ptr(const EdgeSrc& s, int64_t i) {
    return i < s.num_edges ? s.row + i : s.col + (i - s.num_edges);
}
__device__ __forceinline__ const int64_t* src_col_ptr(const EdgeSrc& s, int64_t i) {
    return i < s.num_edges ? s.col + i : s.row + (i - s.num_edges);
}

// How a pass reads entry i: the previous pass's keys, or (first pass) the
// caller's arrays, both ids or the col id alone when the pass's digits lie in
// the col field (row ids are then checked by the first scatter pass, which
// reads both).  Entry i of the (optionally symmetrized) list is (row[i],
// col[i]) for i < num_edges, else the reversed pair of entry i - num_edges;
// its key is row << cbits | col.
enum class Src { kKeys, kBoth, kCol };

template <typename Store, Src kSrc, typename KeyT = typename Store::K>
__device__ __forceinline__ KeyT read_entry(const EdgeSrc& s, const Store& keys, int64_t i,
                                           bool& bad) {
    if (kSrc == Src::kKeys) return keys.load(i);
    const KeyT c = static_cast<KeyT>(clamp_id(*src_col_ptr(s, i), s.num_nodes, bad));
    if (kSrc == Src::kCol) return c;
    const KeyT r = static_cast<KeyT>(clamp_id(*src_row_ptr(s, i), s.num_nodes, bad));
    return (r << s.cbits) | c;
}

// A thread's entries base + q * stride (q < kItems), every load issued before
// any value is used: an index at or past `total` reads entry total - 1 (the
// caller ignores those slots), so that no load sits behind a branch.  (Behind
// per-slot branches the compiler waits for each load before the next.)
template <typename Store, Src kSrc, typename KeyT = typename Store::K>
__device__ __forceinline__ void load_slots(KeyT (&key)[kItems], const EdgeSrc& s,
                                           const Store& keys, int64_t base, int stride,
                                           int64_t total, bool& bad) {
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
        const int64_t i = base + static_cast<int64_t>(q) * stride;
        key[q] = read_entry<Store, kSrc>(s, keys, i < total ? i : total - 1, bad);
    }
}

template <typename KeyT>
__device__ __forceinline__ uint32_t digit_of(KeyT k, int shift) {
    return static_cast<uint32_t>(k >> shift) & (kRadix - 1);
}

// Lanes of this wavefront that are active and hold the same digit d.  For
// each bit, the lanes whose bit differs from this lane's are m ^ e, with m
// the wavefront's ballot of the bit and e = 0 or ~0 this lane's bit: OR-ing
// those over the bits leaves the peers as the lanes never marked.  The OR of
// an XOR is one v_bitop3_b32 per 32-bit half (gfx950): truth table index
// S0 * 4 + S1 * 2 + S2 over (S0 = m, S1 = e, S2 = differ), value
// S2 | (S0 ^ S1).  With the sign-extended bit e as the ballot's operand a bit
// costs four VALU instructions.
constexpr uint32_t bitop3_table_or_xor() {
    uint32_t t = 0;
    for (int i = 0; i < 8; ++i)
        if ((i & 1) | (((i >> 2) ^ (i >> 1)) & 1)) t |= 1u << i;
    return t;
}
static_assert(bitop3_table_or_xor() == 0xbe, "S2 | (S0 ^ S1)");

__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool active) {
    uint32_t differ_lo = 0, differ_hi = 0;
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        const uint32_t e = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int32_t>(d), b, 1));
        const uint64_t m = __builtin_amdgcn_uicmp(e, 0u, 33);  // 33: not equal
        differ_lo = __builtin_amdgcn_bitop3_b32(static_cast<uint32_t>(m), e, differ_lo,
                                                bitop3_table_or_xor());
        differ_hi = __builtin_amdgcn_bitop3_b32(static_cast<uint32_t>(m >> 32), e, differ_hi,
                                                bitop3_table_or_xor());
    }
    const uint64_t act = __ballot(active);
    return act & ~((static_cast<uint64_t>(differ_hi) << 32) | differ_lo);
}

template <int kOp>
__device__ __forceinline__ int64_t op_apply(int64_t a, int64_t b) {
    return kOp == kOpSum ? a + b : (a < b ? a : b);
}

template <int kOp>
__device__ __forceinline__ int64_t op_identity() {
    return kOp == kOpSum ? 0 : INT64_MAX;
}

// Exclusive scan of one value per thread over a block of kThreads threads,
// in thread order.  `wtot` is kThreads / 64 words of LDS.  Returns the
// exclusive prefix; *total (if given) receives the block's reduction.
// Contains two __syncthreads.
template <int kOp, int kThreads = kBlock>
__device__ int64_t block_exclusive_scan(int64_t v, int64_t* wtot, int64_t* total = nullptr) {
    const int lane = __lane_id();
    const int w = threadIdx.x / kWave;
    int64_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int64_t u = __shfl_up(inc, o, kWave);
        if (lane >= o) inc = op_apply<kOp>(inc, u);
    }
    if (lane == kWave - 1) wtot[w] = inc;
    __syncthreads();
    int64_t before = op_identity<kOp>();
    for (int k = 0; k < w; ++k) before = op_apply<kOp>(before, wtot[k]);
    int64_t all = op_identity<kOp>();
    for (int k = 0; k < kThreads / kWave; ++k) all = op_apply<kOp>(all, wtot[k]);
    int64_t excl = __shfl_up(inc, 1, kWave);
    if (lane == 0) excl = op_identity<kOp>();
    if (total) *total = all;
    __syncthreads();
    return op_apply<kOp>(before, excl);
}

// ------------------------------------------------------------- radix pass

// Tile of radix block b.  Workgroups are dispatched to the 8 XCDs round
// robin, and each XCD has its own L2.  Neighbouring tiles share 128-byte
// lines: in the scatter, tile t's run of digit d ends where tile t + 1's run
// of d begins; in the digit counts (digit-major), tiles t .. t + 15 of a digit
// fill one line.  Giving each XCD a contiguous range of tiles puts those
// partial writes (and the scatter's reads of the counts) into one L2.
#ifndef MLXC_CSR_XCD_REMAP
#define MLXC_CSR_XCD_REMAP 1
#endif
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t tiles) {
    if (!MLXC_CSR_XCD_REMAP) return b;
    const int64_t q = tiles / kXcds, r = tiles % kXcds;
    const int64_t x = b % kXcds, i = b / kXcds;  // XCD x runs its i-th block
    // XCDs 0 .. r-1 take q + 1 tiles, the others q: a bijection of [0, tiles)
    return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Per 8192-key tile, the counts of its 256 digits.  The first pass reads the
// caller's arrays; later passes read the digit bytes the previous scatter
// wrote beside the keys (1 byte per key instead of 4 or 8), one 16-byte load
// per thread.  The byte array is padded to whole tiles.
template <typename Store, bool kFirst>
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(EdgeSrc src,
                                                                  const uint8_t* __restrict__ digits,
                                                                  int shift, int64_t total,
                                                                  int64_t tiles,
                                                                  int64_t* __restrict__ hist,
                                                                  int64_t* __restrict__ work) {
    __shared__ int32_t cnt[kSortWaves][kRadix];
    __shared__ int32_t sub[kFirst ? 1 : kSortWaves][kRadix][4];
    const int t = threadIdx.x, w = t / kWave, lane = t % kWave;
    for (int k = t; k < kSortWaves * kRadix; k += kSortThreads) (&cnt[0][0])[k] = 0;
    if (!kFirst)
        for (int k = t; k < kSortWaves * kRadix * 4; k += kSortThreads) (&sub[0][0][0])[k] = 0;
    const int64_t tile = xcd_tile(blockIdx.x, tiles);
    bool bad = false;
    // Counts do not depend on order, so plain LDS atomics do.
    if (kFirst) {
        // all loads first, so that the whole tile is in flight at once
        const int64_t base = tile * kSortTile + w * kWaveTile + lane;
        typename Store::K key[kItems];
        if (shift + kRadixBits <= src.cbits)
            load_slots<Store, Src::kCol>(key, src, Store{}, base, kWave, total, bad);
        else
            load_slots<Store, Src::kBoth>(key, src, Store{}, base, kWave, total, bad);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kItems; ++s) {
            if (base + static_cast<int64_t>(s) * kWave < total)
                atomicAdd(&cnt[w][digit_of(key[s], shift)], 1);
        }
    } else {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const int64_t at = tile * kSortTile + static_cast<int64_t>(t) * kItems;
        const u32x4 v = *reinterpret_cast<const u32x4*>(digits + at);
        __syncthreads();
        // Lanes of a wavefront that add to one LDS word are serialized, and
        // the digits of R-MAT keys are skewed (a tenth of the high digits are
        // 0): four interleaved copies per wavefront, by lane % 4, cut those
        // collisions (0.18 -> 0.15 ms per pass at 2^28 keys).
        int32_t* mine = &sub[w][0][lane & 3];
#pragma unroll
        for (int q = 0; q < kItems; ++q) {
            if (at + q < total) atomicAdd(&mine[4 * ((v[q / 4] >> (8 * (q % 4))) & 0xffu)], 1);
        }
        __syncthreads();
        if (t < kRadix) {
            for (int k = 0; k < kSortWaves; ++k)
                cnt[k][t] = sub[k][t][0] + sub[k][t][1] + sub[k][t][2] + sub[k][t][3];
        }
    }
    __syncthreads();
    if (t < kRadix) {
        int32_t sum = 0;
        for (int k = 0; k < kSortWaves; ++k) sum += cnt[k][t];
        hist[static_cast<int64_t>(t) * tiles + tile] = sum;
    }
    if (kFirst && bad)
        atomicOr(reinterpret_cast<unsigned long long*>(work),
                 static_cast<unsigned long long>(MLXC_STATUS_BAD_NODE));
}

// Two blocks per CU (their LDS fits): at most 128 VGPRs.
template <typename Store, bool kFirst>
__global__ __launch_bounds__(kSortThreads) __attribute__((amdgpu_waves_per_eu(4))) void radix_scatter_kernel(
    EdgeSrc src, Store keys_in, Store keys_out, int shift,
    int64_t total, int64_t tiles, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ digit_totals, int64_t* __restrict__ work,
    uint8_t* __restrict__ next_digits, int next_shift) {
    using KeyT = typename Store::K;
    __shared__ KeyT buf[kSortTile];
    __shared__ int32_t cnt[kSortWaves][kRadix];
    __shared__ int64_t goff[kRadix];
    __shared__ int64_t wtot[kSortWaves];
    const int t = threadIdx.x, w = t / kWave, lane = t % kWave;
    const int64_t tile = xcd_tile(blockIdx.x, tiles);
    for (int k = t; k < kSortWaves * kRadix; k += kSortThreads) (&cnt[0][0])[k] = 0;
    if (t < kRadix) goff[t] = offsets[static_cast<int64_t>(t) * tiles + tile];
    // read now, used after the ranking: the load overlaps the key loads
    const int64_t dtot = digit_totals && t < kRadix ? digit_totals[t] : 0;
    __syncthreads();

    // Rank of every key among the keys of its digit that come before it in
    // this tile's order (wavefront, then slot, then lane): stable.
    const int64_t base = tile * kSortTile + w * kWaveTile + lane;
    KeyT key[kItems];
    int32_t pos[kItems];
    bool bad = false;
    if (kFirst)
        load_slots<Store, Src::kBoth>(key, src, keys_in, base, kWave, total, bad);
    else
        load_slots<Store, Src::kKeys>(key, src, keys_in, base, kWave, total, bad);
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const bool active = base + static_cast<int64_t>(s) * kWave < total;
        const KeyT k = key[s];
        const uint32_t d = digit_of(k, shift);
        const uint64_t peers = match_digit(d, active);
        const int32_t before = cnt[w][d];
        const int rank = lane_rank(peers);
        pos[s] = before + rank;
        if (active && rank == 0) cnt[w][d] = before + __popcll(peers);  // the lowest such lane
    }
    __syncthreads();

    // Thread t < 256 owns digit t: its first position in the reordered tile,
    // and the first position of each wavefront's keys of that digit.
    // offsets[] holds each tile's position inside its digit's output range;
    // the ranges start at the exclusive prefix of digit_totals (with no
    // digit_totals, offsets[] holds the whole position).  Both
    // prefixes come from one scan: the tile counts (at most kSortTile, whose
    // sum fits kTileBits) in the low bits, the digit totals above them.
    constexpr int kTileBits = 14;
    static_assert(kSortTile < (1 << kTileBits), "tile counts fit the low field");
    int32_t c[kSortWaves];
    int32_t tot = 0;
    int64_t packed = 0;
    if (t < kRadix) {
#pragma unroll
        for (int k = 0; k < kSortWaves; ++k) {
            c[k] = cnt[k][t];
            tot += c[k];
        }
        packed = (dtot << kTileBits) | tot;
    }
    const int64_t ex = block_exclusive_scan<kOpSum, kSortThreads>(packed, wtot);
    int32_t at = static_cast<int32_t>(ex & ((1 << kTileBits) - 1));
    if (t < kRadix) {
        // output position of tile entry j of digit t: goff[t] + j
        goff[t] += (ex >> kTileBits) - at;
#pragma unroll
        for (int k = 0; k < kSortWaves; ++k) {
            cnt[k][t] = at;
            at += c[k];
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const int64_t i = base + static_cast<int64_t>(s) * kWave;
        if (i < total) buf[cnt[w][digit_of(key[s], shift)] + pos[s]] = key[s];
    }
    __syncthreads();

    // Consecutive entries of one digit go to consecutive output positions.
    const int64_t left = total - tile * kSortTile;
    const int n = left < kSortTile ? static_cast<int>(left) : kSortTile;
    // With next_digits, each key's digit of the next pass goes beside it.
    for (int j = t; j < n; j += kSortThreads) {
        const KeyT k = buf[j];
        const int64_t at = goff[digit_of(k, shift)] + j;
        keys_out.store(at, k);
        if (next_digits) next_digits[at] = static_cast<uint8_t>(digit_of(k, next_shift));
    }
    if (kFirst && bad)
        atomicOr(reinterpret_cast<unsigned long long*>(work),
                 static_cast<unsigned long long>(MLXC_STATUS_BAD_NODE));
}

// ------------------------------------------------------------- device scan

// Exclusive sum scan of each of gridDim.x rows of len values, in place, one
// block per row; totals[row] <- the row's sum.  The digit counts are 256 such
// rows (digit-major), so one launch replaces the three of a scan over the
// whole array.  Each chunk's loads are issued before the previous chunk is
// scanned.
__global__ __launch_bounds__(kBlock) void row_scan_kernel(int64_t* __restrict__ data, int64_t len,
                                                          int64_t* __restrict__ totals) {
    __shared__ int64_t vals[kChunk + kChunk / kItems];
    __shared__ int64_t wtot[kWaves];
    const int t = threadIdx.x;
    int64_t* row = data + static_cast<int64_t>(blockIdx.x) * len;
    auto slot = [](int j) { return j + j / kItems; };
    int64_t next[kItems];
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const int64_t j = s * kBlock + t;
        next[s] = j < len ? row[j] : 0;
    }
    int64_t carry = 0;
    for (int64_t base = 0; base < len; base += kChunk) {
#pragma unroll
        for (int s = 0; s < kItems; ++s) vals[slot(s * kBlock + t)] = next[s];
        __syncthreads();
        if (base + kChunk < len) {
#pragma unroll
            for (int s = 0; s < kItems; ++s) {
                const int64_t j = base + kChunk + s * kBlock + t;
                next[s] = j < len ? row[j] : 0;
            }
        }
        int64_t run = 0;
#pragma unroll
        for (int s = 0; s < kItems; ++s) run += vals[slot(t * kItems + s)];
        int64_t total;
        int64_t acc = carry + block_exclusive_scan<kOpSum>(run, wtot, &total);
#pragma unroll
        for (int s = 0; s < kItems; ++s) {
            const int j = slot(t * kItems + s);
            const int64_t v = vals[j];
            vals[j] = acc;
            acc += v;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kItems; ++s) {
            const int64_t j = base + s * kBlock + t;
            if (j < len) row[j] = vals[slot(s * kBlock + t)];
        }
        carry += total;
        __syncthreads();
    }
    if (t == 0) totals[blockIdx.x] = carry;
}
// In place over n int64 values, chunks of kChunk per block.  kRev scans from
// the end (logical element j is data[n - 1 - j]).

template <int kOp, bool kRev>
__device__ __forceinline__ int64_t scan_load(const int64_t* data, int64_t n, int64_t j) {
    if (j >= n) return op_identity<kOp>();
    return data[kRev ? n - 1 - j : j];
}

template <int kOp, bool kRev>
__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(const int64_t* __restrict__ data,
                                                             int64_t n,
                                                             int64_t* __restrict__ sums) {
    __shared__ int64_t wtot[kWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
    int64_t acc = op_identity<kOp>();
    for (int s = 0; s < kItems; ++s)
        acc = op_apply<kOp>(acc, scan_load<kOp, kRev>(data, n, base + s * kBlock + threadIdx.x));
    int64_t total;
    block_exclusive_scan<kOp>(acc, wtot, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Up to this many chunks, each block of scan_down_kernel reduces the chunk
// sums of the blocks before it itself (at most kScanFlatChunks values, read
// from L2), so no launch has to scan the sums in between.  That costs
// chunks^2 / 2 loads in all; above it the sums are scanned first (by the same
// two launches, one level up) and each block reads its own carry.
constexpr int64_t kScanFlatChunks = 4096;

// kPre: sums[b] already holds the exclusive scan of the chunk sums before
// chunk b.  Otherwise each block reduces sums[0 .. b) itself.  The last block
// writes the whole reduction to *total_out (if given).
template <int kOp, bool kRev, bool kExcl, bool kPre>
__global__ __launch_bounds__(kBlock) void scan_down_kernel(int64_t* __restrict__ data, int64_t n,
                                                           const int64_t* __restrict__ sums,
                                                           int64_t* __restrict__ total_out) {
    // Padded so that thread t's 16 consecutive values sit in distinct banks.
    __shared__ int64_t vals[kChunk + kChunk / kItems];
    __shared__ int64_t wtot[kWaves];
    const int t = threadIdx.x;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
    auto slot = [](int j) { return j + j / kItems; };
    for (int s = 0; s < kItems; ++s) {
        const int j = s * kBlock + t;
        vals[slot(j)] = scan_load<kOp, kRev>(data, n, base + j);
    }
    int64_t carry;
    if (kPre) {
        carry = sums[blockIdx.x];
        __syncthreads();  // covers vals
    } else {
        int64_t part = op_identity<kOp>();
        for (int64_t k = t; k < blockIdx.x; k += kBlock) part = op_apply<kOp>(part, sums[k]);
        block_exclusive_scan<kOp>(part, wtot, &carry);  // its two barriers also cover vals
    }
    int64_t run = op_identity<kOp>();
    for (int s = 0; s < kItems; ++s) run = op_apply<kOp>(run, vals[slot(t * kItems + s)]);
    int64_t own;
    int64_t acc = op_apply<kOp>(carry, block_exclusive_scan<kOp>(run, wtot, &own));
    if (total_out && t == 0 && blockIdx.x == gridDim.x - 1) *total_out = op_apply<kOp>(carry, own);
    for (int s = 0; s < kItems; ++s) {
        const int j = slot(t * kItems + s);
        const int64_t v = vals[j];
        if (kExcl) {
            vals[j] = acc;
            acc = op_apply<kOp>(acc, v);
        } else {
            acc = op_apply<kOp>(acc, v);
            vals[j] = acc;
        }
    }
    __syncthreads();
    for (int s = 0; s < kItems; ++s) {
        const int64_t j = base + s * kBlock + t;
        if (j < n) data[kRev ? n - 1 - j : j] = vals[slot(s * kBlock + t)];
    }
}

// ------------------------------------------------------------- finish

__global__ void fill_words_kernel(int64_t* __restrict__ out, int64_t n,
                                  const int64_t* __restrict__ value) {
    const int64_t v = *value;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = v;
}

__global__ void set_word_kernel(int64_t* __restrict__ word, int64_t v) {
    if (threadIdx.x == 0) *word = v;
}

// key[s] = keys[i], prev[s] = keys[i - 1] for i = chunk + s * kBlock + t (the
// block's kChunk entries from `chunk`), the keys' loads all issued before any
// is used (indices clamped into [0, total); the caller ignores slots with
// i >= total, and prev of i = 0).  prev is thread t - 1's key of the slot: a
// lane shuffle inside a wavefront, `edge` (kItems x kWaves words of LDS) for
// lane 0, and one more load for the chunk's first entry.  Contains a barrier.
template <typename Store, typename KeyT = typename Store::K>
__device__ __forceinline__ void load_pairs(KeyT (&key)[kItems], KeyT (&prev)[kItems],
                                           const Store& keys, int64_t chunk, int64_t total,
                                           KeyT (*edge)[kWaves]) {
    const int t = threadIdx.x, w = t / kWave, lane = t % kWave;
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const int64_t i = chunk + s * kBlock + t;
        key[s] = keys.load(i < total ? i : total - 1);
    }
    const int64_t i0 = chunk > 0 ? (chunk - 1 < total ? chunk - 1 : total - 1) : 0;
    const KeyT first_prev = keys.load(i0);
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        prev[s] = __shfl_up(key[s], 1, kWave);
        if (lane == kWave - 1) edge[s][w] = key[s];
    }
    __syncthreads();
    if (lane == 0) {
#pragma unroll
        for (int s = 0; s < kItems; ++s)
            prev[s] = w > 0 ? edge[s][w - 1] : s > 0 ? edge[s - 1][kWaves - 1] : first_prev;
    }
}

// counts[chunk] <- kept entries of chunk (kChunk entries).
template <typename Store>
__global__ __launch_bounds__(kBlock) void dedup_count_kernel(Store keys,
                                                             int64_t total,
                                                             int64_t* __restrict__ counts) {
    __shared__ int64_t wtot[kWaves];
    __shared__ typename Store::K edge[kItems][kWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
    typename Store::K key[kItems], prev[kItems];
    load_pairs(key, prev, keys, static_cast<int64_t>(blockIdx.x) * kChunk, total, edge);
    int64_t c = 0;
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const int64_t i = base + s * kBlock;
        c += i < total && (i == 0 || prev[s] != key[s]);
    }
    int64_t all;
    block_exclusive_scan<kOpSum>(c, wtot, &all);
    if (threadIdx.x == 0) counts[blockIdx.x] = all;
}

// Writes col[p] for every kept entry (p = its rank among kept entries) and
// rowptr[row] = p at the first entry of each row present.  kDedup: the
// chunk's first p comes from chunk_base (the exclusive scan of
// dedup_count_kernel's counts).
template <typename Store, bool kDedup>
__global__ __launch_bounds__(kBlock) void csr_emit_kernel(Store keys,
                                                          int64_t total, int cbits,
                                                          const int64_t* __restrict__ chunk_base,
                                                          int64_t* __restrict__ rowptr,
                                                          int64_t* __restrict__ col_out) {
    using KeyT = typename Store::K;
    __shared__ int32_t wkept[kItems][kWaves];
    const int t = threadIdx.x, w = t / kWave;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
    const KeyT cmask = cbits == 0 ? KeyT(0) : (~KeyT(0) >> (8 * sizeof(KeyT) - cbits));
    __shared__ KeyT edge[kItems][kWaves];
    KeyT key[kItems], before[kItems];
    load_pairs(key, before, keys, base, total, edge);
    uint32_t keep_bits = 0, start_bits = 0;
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        const int64_t i = base + s * kBlock + t;
        const bool valid = i < total;
        const KeyT k = key[s], prev = before[s];
        const bool keep = valid && (!kDedup || i == 0 || prev != k);
        const bool row_start = valid && (i == 0 || (prev >> cbits) != (k >> cbits));
        keep_bits |= static_cast<uint32_t>(keep) << s;
        start_bits |= static_cast<uint32_t>(row_start) << s;
        if (kDedup) {
            const uint64_t m = __ballot(keep);
            if (__lane_id() == 0) wkept[s][w] = __popcll(m);
        }
    }
    int64_t p0 = base;
    if (kDedup) {
        __syncthreads();
        p0 = chunk_base[blockIdx.x];
        // entries before slot 0 of this wavefront: earlier wavefronts of slot 0
        for (int k = 0; k < w; ++k) p0 += wkept[0][k];
    }
#pragma unroll
    for (int s = 0; s < kItems; ++s) {
        int64_t p;
        if (kDedup) {
            const bool keep = (keep_bits >> s) & 1u;
            p = p0 + lane_rank(__ballot(keep));
            // advance p0 to slot s + 1 of this wavefront: the rest of slot s
            // (this and later wavefronts), then earlier wavefronts of s + 1
            for (int k = w; k < kWaves; ++k) p0 += wkept[s][k];
            if (s + 1 < kItems)
                for (int k = 0; k < w; ++k) p0 += wkept[s + 1][k];
        } else {
            p = base + s * kBlock + t;
        }
        if ((keep_bits >> s) & 1u) {
            const KeyT k = key[s];
            col_out[p] = static_cast<int64_t>(k & cmask);
            if ((start_bits >> s) & 1u) rowptr[static_cast<int64_t>(k >> cbits)] = p;
        }
    }
}

// ------------------------------------------------------------- host side

int bits_for(int64_t num_nodes) {
    int b = 0;
    for (uint64_t x = num_nodes > 1 ? static_cast<uint64_t>(num_nodes - 1) : 0; x; x >>= 1) ++b;
    return b;
}

size_t round256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct CsrLayout {
    int64_t total = 0;  // entries to sort
    int cbits = 0;
    int passes = 0;
    int key_bytes = 4;   // 4, 5 (Keys40), 6 (Keys48) or 8
    int64_t tiles = 0;   // radix tiles of kSortTile keys
    int64_t chunks = 0;  // finish chunks of kChunk keys
    size_t keys[2] = {0, 0};  // the two key arrays (Keys40 / Keys48: low halves)
    size_t keys_hi[2] = {0, 0};  // Keys40 / Keys48: the high bits
    size_t digits = 0, hist = 0, totals = 0, sums = 0, bytes = 0;
};

// Words of chunk sums device_scan needs for n values: one per chunk, plus
// those of the sums' own scan when it takes the levelled form.
int64_t scan_sums_words(int64_t n) {
    const int64_t chunks = (n + kChunk - 1) / kChunk;
    return chunks + (chunks > kScanFlatChunks ? scan_sums_words(chunks) : 0);
}

CsrLayout csr_layout(int64_t num_nodes, int64_t num_edges, int32_t flags) {
    CsrLayout l;
    l.total = (flags & MLXC_CSR_SYMMETRIZE) ? 2 * num_edges : num_edges;
    l.cbits = bits_for(num_nodes);
    const int key_bits = 2 * l.cbits;
    l.key_bytes = key_bits <= 32 ? 4 : key_bits <= 40 ? 5 : key_bits <= 48 ? 6 : 8;
    l.passes = key_bits == 0 ? 1 : (key_bits + kRadixBits - 1) / kRadixBits;
    l.tiles = (l.total + kSortTile - 1) / kSortTile;
    l.chunks = (l.total + kChunk - 1) / kChunk;
    const size_t n = static_cast<size_t>(l.total);
    // the digit counts, and after the last pass the finish chunks' counts
    int64_t hist_n = kRadix * l.tiles;
    if (l.chunks > hist_n) hist_n = l.chunks;
    int64_t scan_n = hist_n;
    if (num_nodes + 1 > scan_n) scan_n = num_nodes + 1;
    const int64_t sum_words = scan_sums_words(scan_n);
    size_t at = round256(MLXC_WORK_WORDS * sizeof(int64_t));
    for (int b = 0; b < 2; ++b) {
        const bool split = l.key_bytes == 5 || l.key_bytes == 6;
        l.keys[b] = at;
        at += round256(n * (split ? 4 : l.key_bytes));
        if (split) {
            l.keys_hi[b] = at;
            at += round256(n * (l.key_bytes - 4));
        }
    }
    l.digits = at;  // the next pass's digit of each key, padded to whole tiles
    at += round256(static_cast<size_t>(l.tiles) * kSortTile);
    l.hist = at;
    at += round256(static_cast<size_t>(hist_n) * sizeof(int64_t));
    l.totals = at;  // the digit totals of a pass
    at += round256(kRadix * sizeof(int64_t));
    l.sums = at;
    at += round256(static_cast<size_t>(sum_words + 1) * sizeof(int64_t));
    l.bytes = at;
    return l;
}

// Up to this many values, one block scans faster than the two launches of
// device_scan.
#ifndef MLXC_ROW_SCAN_MAX
#define MLXC_ROW_SCAN_MAX (4 * kChunk)
#endif
constexpr int64_t kRowScanMax = MLXC_ROW_SCAN_MAX;
// The digit counts are scanned by rows (one block per digit) up to this many
// tiles per row.
#ifndef MLXC_ROW_SCAN_TILES
#define MLXC_ROW_SCAN_TILES kChunk
#endif
constexpr int64_t kRowScanTiles = MLXC_ROW_SCAN_TILES;

// Scan of n int64 values in place: two launches up to kScanFlatChunks
// chunks of kChunk values, and two more per level of chunk sums above that.
// `sums` holds scan_sums_words(n) words.
template <int kOp, bool kRev, bool kExcl>
int device_scan(int64_t* data, int64_t n, int64_t* sums, int64_t* total_out, hipStream_t s) {
    if (n <= 0) return MLXC_OK;
    const int64_t chunks = (n + kChunk - 1) / kChunk;
    hipLaunchKernelGGL((scan_reduce_kernel<kOp, kRev>), dim3(chunks), dim3(kBlock), 0, s, data, n,
                       sums);
    MLXC_HIP_TRY(hipGetLastError());
    if (chunks <= kScanFlatChunks) {
        hipLaunchKernelGGL((scan_down_kernel<kOp, kRev, kExcl, false>), dim3(chunks), dim3(kBlock),
                           0, s, data, n, sums, total_out);
    } else {
        // the chunk sums, exclusive and in chunk order, with the next level's
        // sums after them
        if (int rc = device_scan<kOp, false, true>(sums, chunks, sums + chunks, nullptr, s))
            return rc;
        hipLaunchKernelGGL((scan_down_kernel<kOp, kRev, kExcl, true>), dim3(chunks), dim3(kBlock),
                           0, s, data, n, sums, total_out);
    }
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int fill_words(int64_t* out, int64_t n, const int64_t* value, hipStream_t s) {
    int grid = 0;
    if (int rc = stream_grid(n, 8, grid)) return rc;
    hipLaunchKernelGGL(fill_words_kernel, dim3(grid), dim3(kBlock), 0, s, out, n, value);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

Keys32 key_store(char* ws, const CsrLayout& l, int b, Keys32) {
    return Keys32{reinterpret_cast<uint32_t*>(ws + l.keys[b])};
}
Keys40 key_store(char* ws, const CsrLayout& l, int b, Keys40) {
    return Keys40{reinterpret_cast<uint32_t*>(ws + l.keys[b]),
                  reinterpret_cast<uint8_t*>(ws + l.keys_hi[b])};
}
Keys48 key_store(char* ws, const CsrLayout& l, int b, Keys48) {
    return Keys48{reinterpret_cast<uint32_t*>(ws + l.keys[b]),
                  reinterpret_cast<uint16_t*>(ws + l.keys_hi[b])};
}
Keys64 key_store(char* ws, const CsrLayout& l, int b, Keys64) {
    return Keys64{reinterpret_cast<uint64_t*>(ws + l.keys[b])};
}

template <typename Store>
int csr_build_typed(const EdgeSrc& src, const CsrLayout& l, int32_t flags, int64_t* rowptr,
                    int64_t* col_out, char* ws, hipStream_t s) {
    int64_t* work = reinterpret_cast<int64_t*>(ws);
    const Store buf[2] = {key_store(ws, l, 0, Store{}), key_store(ws, l, 1, Store{})};
    int64_t* hist = reinterpret_cast<int64_t*>(ws + l.hist);
    int64_t* totals = reinterpret_cast<int64_t*>(ws + l.totals);
    int64_t* sums = reinterpret_cast<int64_t*>(ws + l.sums);
    uint8_t* digits = reinterpret_cast<uint8_t*>(ws + l.digits);
    Store in{};
    for (int p = 0; p < l.passes; ++p) {
        const int shift = p * kRadixBits;
        const Store out = buf[p & 1];
        uint8_t* next_digits = p + 1 < l.passes ? digits : nullptr;
        if (p == 0)
            hipLaunchKernelGGL((radix_hist_kernel<Store, true>), dim3(l.tiles), dim3(kSortThreads), 0, s,
                               src, digits, shift, l.total, l.tiles, hist, work);
        else
            hipLaunchKernelGGL((radix_hist_kernel<Store, false>), dim3(l.tiles), dim3(kSortThreads), 0, s,
                               src, digits, shift, l.total, l.tiles, hist, work);
        MLXC_HIP_TRY(hipGetLastError());
        // short rows: one block per digit; long rows: a scan of the whole
        // array, which spreads each row over many blocks
        const bool by_rows = l.tiles <= kRowScanTiles;
        if (by_rows)
            hipLaunchKernelGGL(row_scan_kernel, dim3(kRadix), dim3(kBlock), 0, s, hist, l.tiles,
                               totals);
        else if (int rc = device_scan<kOpSum, false, true>(hist, kRadix * l.tiles, sums, nullptr, s))
            return rc;
        const int64_t* digit_totals = by_rows ? totals : nullptr;
        if (p == 0)
            hipLaunchKernelGGL((radix_scatter_kernel<Store, true>), dim3(l.tiles), dim3(kSortThreads), 0,
                               s, src, in, out, shift, l.total, l.tiles, hist, digit_totals, work,
                               next_digits, shift + kRadixBits);
        else
            hipLaunchKernelGGL((radix_scatter_kernel<Store, false>), dim3(l.tiles), dim3(kSortThreads), 0,
                               s, src, in, out, shift, l.total, l.tiles, hist, digit_totals, work,
                               next_digits, shift + kRadixBits);
        MLXC_HIP_TRY(hipGetLastError());
        in = out;
    }
    // work[1] <- entries kept; rowptr <- that count everywhere, then the row
    // starts, then the reverse min-scan.  The digit counts' space holds the
    // finish chunks' counts.
    const int64_t chunks = l.chunks;
    int64_t* chunk_base = hist;
    if (flags & MLXC_CSR_DEDUP) {
        hipLaunchKernelGGL((dedup_count_kernel<Store>), dim3(chunks), dim3(kBlock), 0, s, in,
                           l.total, chunk_base);
        MLXC_HIP_TRY(hipGetLastError());
        if (chunks <= kRowScanMax) {
            hipLaunchKernelGGL(row_scan_kernel, dim3(1), dim3(kBlock), 0, s, chunk_base, chunks,
                               work + 1);
        } else if (int rc = device_scan<kOpSum, false, true>(chunk_base, chunks, sums, work + 1, s)) {
            return rc;
        }
    } else {
        hipLaunchKernelGGL(set_word_kernel, dim3(1), dim3(kWave), 0, s, work + 1, l.total);
    }
    MLXC_HIP_TRY(hipGetLastError());
    if (int rc = fill_words(rowptr, src.num_nodes + 1, work + 1, s)) return rc;
    if (flags & MLXC_CSR_DEDUP)
        hipLaunchKernelGGL((csr_emit_kernel<Store, true>), dim3(chunks), dim3(kBlock), 0, s, in,
                           l.total, l.cbits, chunk_base, rowptr, col_out);
    else
        hipLaunchKernelGGL((csr_emit_kernel<Store, false>), dim3(chunks), dim3(kBlock), 0, s, in,
                           l.total, l.cbits, chunk_base, rowptr, col_out);
    MLXC_HIP_TRY(hipGetLastError());
    return device_scan<kOpMin, true, false>(rowptr, src.num_nodes + 1, sums, nullptr, s);
}

}  // namespace

size_t csr_build_workspace_bytes(int64_t num_nodes, int64_t num_edges, int32_t flags) {
    return csr_layout(num_nodes, num_edges, flags).bytes;
}

int launch_csr_build(const int64_t* row, const int64_t* col, int64_t num_edges, int64_t num_nodes,
                     int32_t flags, int64_t* rowptr, int64_t* col_out, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
    const CsrLayout l = csr_layout(num_nodes, num_edges, flags);
    if (workspace_bytes < l.bytes)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "workspace smaller than mlxc_csr_build_workspace_bytes()");
    char* ws = static_cast<char*>(workspace);
    int64_t* work = reinterpret_cast<int64_t*>(ws);
    if (int rc = launch_zero_work(work, stream)) return rc;
    if (l.total == 0) return fill_words(rowptr, num_nodes + 1, work + 1, stream);
    const EdgeSrc src{row, col, num_edges, num_nodes, l.cbits};
    if (l.key_bytes == 4) return csr_build_typed<Keys32>(src, l, flags, rowptr, col_out, ws, stream);
    if (l.key_bytes == 5) return csr_build_typed<Keys40>(src, l, flags, rowptr, col_out, ws, stream);
    if (l.key_bytes == 6) return csr_build_typed<Keys48>(src, l, flags, rowptr, col_out, ws, stream);
    return csr_build_typed<Keys64>(src, l, flags, rowptr, col_out, ws, stream);
}

}  // namespace mlxc
