// Skip-gram context windows over walks: the consumer right after the walk in
// node2vec training.  Not part of the reference (it stops at the walks,
// /root/reference/random_walks/BiasedRandomWalk.cpp:96); the layout follows
// torch_geometric's Node2Vec.pos_sample / neg_sample:
//   W = walk_nodes - context_size + 1 windows per walk, window-major:
//   out[(j * N + n) * C + k] = walk[n][j + k],  j < W, k < C.
// Negative windows use the same layout over the walk
//   [start[n], u(n, 1), ..., u(n, L)],  u(n, l) = node drawn uniformly from
//   [0, num_nodes) by Philox4x32-10 (key = seed, counter = (n lo, n hi, l, 0),
//   word 0 x): u = (x * num_nodes) >> 32.
//
// One block serves a tile of walks for every window position j: the tile's
// walk rows are staged in LDS once (one coalesced read), and the stores of one
// j are one contiguous run of tile * C entries.
#include "walk_host.h"

namespace mlxc {

namespace {

constexpr int kWinTile = 64;  // walks per block (at most)
constexpr int kMaxContext = 32;
constexpr int kWinSlots = (kWinTile * kMaxContext + kBlock - 1) / kBlock;
constexpr size_t kTileLds = 64 * 1024;  // LDS bytes for the walk rows of a tile

// Window stores are streamed past the caches: nothing here reads them again.
#ifndef MLXC_WIN_NT
#define MLXC_WIN_NT 1
#endif
template <typename T>
__device__ __forceinline__ void put(T* p, T v) {
#if MLXC_WIN_NT
    __builtin_nontemporal_store(v, p);
#else
    *p = v;
#endif
}

// Writes the windows of the tile's rows (LDS, walk_nodes entries each) for
// every window position j.
template <typename T>
__device__ __forceinline__ void emit_windows(const T* rw, int64_t tile, int64_t n0,
                                             int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                                             T* __restrict__ out);

template <typename T>
__device__ __forceinline__ void emit_windows(const T* rw, int64_t tile, int64_t n0,
                                             int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                                             T* __restrict__ out) {
    const int entries = static_cast<int>(tile) * ctx;  // one window of every walk in the tile
    const int windows = walk_nodes - ctx + 1;
    // this thread's entries of a window position: (walk, offset) pairs
    int32_t src[kWinSlots];
#pragma unroll
    for (int i = 0; i < kWinSlots; ++i) {
        const int e = threadIdx.x + i * kBlock;
        src[i] = e < entries ? (e / ctx) * walk_nodes + e % ctx : -1;
    }
    for (int j = 0; j < windows; ++j) {
        T* o = out + (static_cast<int64_t>(j) * num_walks + n0) * ctx;
#pragma unroll
        for (int i = 0; i < kWinSlots; ++i)
            if (src[i] >= 0) put(o + threadIdx.x + i * kBlock, rw[src[i] + j]);
    }
}

// `per_block` walks per block (<= kWinTile), so that their rows fit kTileLds
// bytes of LDS.
template <typename T>
__global__ __launch_bounds__(kBlock) void context_windows_kernel(const T* __restrict__ walks,
                                                                 int64_t num_walks,
                                                                 int32_t walk_nodes, int32_t ctx,
                                                                 int32_t per_block,
                                                                 T* __restrict__ out) {
    extern __shared__ unsigned char smem[];
    T* rw = reinterpret_cast<T*>(smem);
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t tile = num_walks - n0 < per_block ? num_walks - n0 : per_block;
    const int cells = static_cast<int>(tile) * walk_nodes;
    const T* in = walks + n0 * walk_nodes;  // the tile's rows are contiguous
    for (int e = threadIdx.x; e < cells; e += kBlock) rw[e] = in[e];
    __syncthreads();
    emit_windows(rw, tile, n0, num_walks, walk_nodes, ctx, out);
}

__device__ __forceinline__ int64_t negative_node(int64_t n, int32_t l, int64_t num_nodes,
                                                 uint32_t k0, uint32_t k1) {
    uint32_t c0 = static_cast<uint32_t>(n), c1 = static_cast<uint32_t>(static_cast<uint64_t>(n) >> 32),
             c2 = static_cast<uint32_t>(l), c3 = 0;
    philox4x32_10(c0, c1, c2, c3, k0, k1);
    return static_cast<int64_t>((static_cast<uint64_t>(c0) * static_cast<uint64_t>(num_nodes)) >> 32);
}

// `per_block` walks per block (<= kWinTile), so that their generated rows fit
// kTileLds bytes of LDS.
template <typename T>
__global__ __launch_bounds__(kBlock) void negative_windows_kernel(
    const int64_t* __restrict__ start, int64_t num_walks, int32_t walk_length, int32_t ctx,
    int64_t num_nodes, uint32_t k0, uint32_t k1, int32_t per_block, T* __restrict__ out) {
    // the tile's walks [start, u_1..u_L] are generated once into LDS
    extern __shared__ unsigned char smem[];
    T* rw = reinterpret_cast<T*>(smem);
    const int walk_nodes = walk_length + 1;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t tile = num_walks - n0 < per_block ? num_walks - n0 : per_block;
    const int cells = static_cast<int>(tile) * walk_nodes;
    for (int e = threadIdx.x; e < cells; e += kBlock) {
        const int w = e / walk_nodes, l = e % walk_nodes;
        const int64_t n = n0 + w;
        rw[e] = static_cast<T>(l == 0 ? start[n] : negative_node(n, l, num_nodes, k0, k1));
    }
    __syncthreads();
    emit_windows(rw, tile, n0, num_walks, walk_nodes, ctx, out);
}

}  // namespace

// Walks per block whose rows of walk_nodes entries fit kTileLds bytes.
int tile_walks(int32_t walk_nodes, size_t esz) {
    const size_t fit = kTileLds / (static_cast<size_t>(walk_nodes) * esz);
    return fit > static_cast<size_t>(kWinTile) ? kWinTile : static_cast<int>(fit);
}

int launch_context_windows(const void* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                           int32_t elem_type, void* out, hipStream_t stream) {
    const size_t esz = elem_type == MLXC_OUT_INT32 ? 4 : 8;
    const int per_block = tile_walks(walk_nodes, esz);
    if (per_block < 1) return fail(MLXC_ERR_INVALID_ARGUMENT, "walks too long for windows");
    const int64_t grid = (num_walks + per_block - 1) / per_block;
    const size_t lds = static_cast<size_t>(per_block) * walk_nodes * esz;
    if (elem_type == MLXC_OUT_INT32)
        hipLaunchKernelGGL(context_windows_kernel<int32_t>, dim3(grid), dim3(kBlock), lds, stream,
                           static_cast<const int32_t*>(walks), num_walks, walk_nodes, ctx,
                           per_block, static_cast<int32_t*>(out));
    else
        hipLaunchKernelGGL(context_windows_kernel<int64_t>, dim3(grid), dim3(kBlock), lds, stream,
                           static_cast<const int64_t*>(walks), num_walks, walk_nodes, ctx,
                           per_block, static_cast<int64_t*>(out));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int windows_max_nodes(int32_t elem_type) {
    return static_cast<int>(kTileLds / (elem_type == MLXC_OUT_INT32 ? 4 : 8));
}

int launch_negative_windows(const int64_t* start, int64_t num_walks, int32_t walk_length,
                            int32_t ctx, int64_t num_nodes, uint64_t seed, int32_t out_type,
                            void* out, hipStream_t stream) {
    const size_t esz = out_type == MLXC_OUT_INT32 ? 4 : 8;
    const int per_block = tile_walks(walk_length + 1, esz);
    if (per_block < 1) return fail(MLXC_ERR_INVALID_ARGUMENT, "walk_length too large");
    const int64_t grid = (num_walks + per_block - 1) / per_block;
    const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
    const size_t lds = static_cast<size_t>(per_block) * (walk_length + 1) * esz;
    if (out_type == MLXC_OUT_INT32)
        hipLaunchKernelGGL(negative_windows_kernel<int32_t>, dim3(grid), dim3(kBlock), lds, stream,
                           start, num_walks, walk_length, ctx, num_nodes, k0, k1, per_block,
                           static_cast<int32_t*>(out));
    else
        hipLaunchKernelGGL(negative_windows_kernel<int64_t>, dim3(grid), dim3(kBlock), lds, stream,
                           start, num_walks, walk_length, ctx, num_nodes, k0, k1, per_block,
                           static_cast<int64_t*>(out));
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

}  // namespace mlxc
