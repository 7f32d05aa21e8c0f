// Random-read probe: the device's ceiling of random reads from a table of a
// given size, the bound of the walk kernels (each walk step is one or two
// dependent reads at random addresses).  Every lane reads loads_per_lane
// addresses per iteration, uniform over the table; with `dependent`, each
// address also depends on the value the same chain loaded the iteration
// before, as a walk's next read depends on the record it just read.  No
// reference counterpart: the reference has no device code for this path.
#include "walk_host.h"

namespace mlxc {

namespace {

constexpr int kProbeBlock = 256;  // threads per block

// 64-bit LCG step (Knuth's MMIX constants); its high 32 bits are the draw.
__device__ __forceinline__ uint64_t lcg(uint64_t x) {
    return x * 6364136223846793005ull + 1442695040888963407ull;
}

template <int kBytes>
struct ProbeLoad;
template <>
struct ProbeLoad<4> {
    __device__ static uint32_t at(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
};
template <>
struct ProbeLoad<16> {
    __device__ static uint32_t at(const uint8_t* p) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        return v.x ^ v.y ^ v.z ^ v.w;
    }
};

// K chains per lane.  Chain k of thread t draws its addresses from its own
// LCG, seeded by (seed, t, k); dependent chains XOR the high word of each
// draw with a mix of the value they loaded last, so the next load waits for
// the previous one.  The XOR of every loaded value goes to *sink only when
// it equals a value no table of random words makes likely, which keeps the
// loads live without storing per thread.
template <int K, int kBytes, bool kDep>
__global__ __launch_bounds__(kProbeBlock) void gather_probe_kernel(const uint8_t* __restrict__ table,
                                                              uint64_t slots, int64_t iterations,
                                                              uint64_t seed,
                                                              uint32_t* __restrict__ sink) {
    const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * kProbeBlock + threadIdx.x;
    uint64_t x[K];
    uint32_t last[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        x[k] = lcg(lcg(seed ^ ((tid * K + k) * 0x9E3779B97F4A7C15ull)));
        last[k] = 0;
    }
    uint32_t acc = 0;
    for (int64_t it = 0; it < iterations; ++it) {
        uint32_t v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            x[k] = lcg(x[k]);
            const uint32_t h = static_cast<uint32_t>(x[k] >> 32) ^ (kDep ? last[k] : 0u);
            const uint64_t slot = (static_cast<uint64_t>(h) * slots) >> 32;
            v[k] = ProbeLoad<kBytes>::at(table + slot * kBytes);
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (kDep) last[k] = v[k] * 0x9E3779B1u;
            acc ^= v[k];
        }
    }
    if (acc == 0x5EEDF00Du) sink[0] = acc;
}

template <int K, int kBytes>
int launch_probe_k(bool dep, dim3 grid, const uint8_t* table, uint64_t slots, int64_t iterations,
                   uint64_t seed, uint32_t* sink, hipStream_t stream) {
    if (dep)
        hipLaunchKernelGGL((gather_probe_kernel<K, kBytes, true>), grid, dim3(kProbeBlock), 0, stream,
                           table, slots, iterations, seed, sink);
    else
        hipLaunchKernelGGL((gather_probe_kernel<K, kBytes, false>), grid, dim3(kProbeBlock), 0, stream,
                           table, slots, iterations, seed, sink);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

template <int kBytes>
int launch_probe_bytes(int k, bool dep, dim3 grid, const uint8_t* table, uint64_t slots,
                       int64_t iterations, uint64_t seed, uint32_t* sink, hipStream_t stream) {
    switch (k) {
    case 1: return launch_probe_k<1, kBytes>(dep, grid, table, slots, iterations, seed, sink, stream);
    case 2: return launch_probe_k<2, kBytes>(dep, grid, table, slots, iterations, seed, sink, stream);
    case 4: return launch_probe_k<4, kBytes>(dep, grid, table, slots, iterations, seed, sink, stream);
    default: return launch_probe_k<8, kBytes>(dep, grid, table, slots, iterations, seed, sink, stream);
    }
}

}  // namespace

int launch_gather_probe(const void* table, int64_t table_bytes, int32_t load_bytes,
                        int32_t loads_per_lane, int32_t dependent, int32_t blocks_per_cu,
                        int64_t iterations, uint64_t seed, uint32_t* sink, int64_t* loads_issued,
                        hipStream_t stream) {
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    const int64_t blocks = static_cast<int64_t>(info.cus) * blocks_per_cu;
    const uint64_t slots = static_cast<uint64_t>(table_bytes / load_bytes);
    *loads_issued = blocks * kProbeBlock * iterations * loads_per_lane;
    const dim3 grid(static_cast<unsigned>(blocks));
    const uint8_t* t = static_cast<const uint8_t*>(table);
    return load_bytes == 4
               ? launch_probe_bytes<4>(loads_per_lane, dependent != 0, grid, t, slots, iterations,
                                       seed, sink, stream)
               : launch_probe_bytes<16>(loads_per_lane, dependent != 0, grid, t, slots,
                                        iterations, seed, sink, stream);
}

}  // namespace mlxc
