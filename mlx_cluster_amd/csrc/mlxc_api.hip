// The C ABI of libmlxc.so (include/mlxc.h): argument validation, workspace
// reset and dispatch to the kernel launchers.  Every entry point checks its
// arguments on the host before touching the device and reports failures as
// a negative code plus a thread-local message.
#include <climits>
#include <cmath>
#include <mutex>
#include <string>

#include "walk_host.h"

// Workspace of mlxc_random_walk_noalloc, one per GPU.  In host code this
// name is only a stand-in for the symbol: kernels get its device address,
// looked up once per device by noalloc_scratch().
static __device__ __align__(256) unsigned char scratch[MLXC_NOALLOC_SCRATCH_BYTES];

namespace mlxc {

namespace {
thread_local std::string g_last_error;
}

thread_local hipEvent_t g_walk_events[2] = {nullptr, nullptr};

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

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

namespace {

int check_workspace(const void* work, size_t work_bytes) {
    if (!work) return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must not be NULL");
    if (work_bytes < MLXC_WORK_WORDS * sizeof(int64_t))
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "workspace must hold at least MLXC_WORK_WORDS int64 words");
    if (reinterpret_cast<uintptr_t>(work) % 16 != 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    return MLXC_OK;
}

// A walk's row holds walk_length + 1 entries, which the kernels count in int32.
int check_walk_length(int32_t walk_length) {
    if (walk_length < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "walk_length must be >= 0");
    if (walk_length == INT32_MAX)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "walk_length must be below 2^31 - 1");
    return MLXC_OK;
}

int check_graph(const int64_t* rowptr, int64_t num_nodes, const int64_t* col, int64_t num_edges,
                const int64_t* start, int64_t num_walks, int32_t walk_length,
                const void* n_out) {
    if (num_nodes < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes must be >= 0");
    if (num_edges < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_edges must be >= 0");
    if (num_walks < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_walks must be >= 0");
    if (int rc = check_walk_length(walk_length)) return rc;
    if (num_walks > 0) {
        if (!rowptr || !start || !n_out)
            return fail(MLXC_ERR_INVALID_ARGUMENT, "rowptr, start and n_out must not be NULL");
        if (num_edges > 0 && !col) return fail(MLXC_ERR_INVALID_ARGUMENT, "col must not be NULL");
        if (num_walks > INT64_MAX / (static_cast<int64_t>(walk_length) + 1))
            return fail(MLXC_ERR_INVALID_ARGUMENT, "num_walks * (walk_length + 1) overflows int64");
    }
    return MLXC_OK;
}

// The output element type, and whether the ids fit it.
int check_out_type(int32_t out_type, int64_t num_nodes, int64_t num_edges, const void* e_out) {
    if (out_type != MLXC_OUT_INT64 && out_type != MLXC_OUT_INT32)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "out_type must be MLXC_OUT_INT64 or MLXC_OUT_INT32");
    if (out_type == MLXC_OUT_INT32 && (num_nodes > INT32_MAX || (e_out && num_edges > INT32_MAX)))
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "MLXC_OUT_INT32 needs num_nodes (and, with edge output, num_edges) below 2^31");
    return MLXC_OK;
}

int check_walk(const int64_t* rowptr, int64_t num_nodes, const int64_t* col, int64_t num_edges,
               const int64_t* start, int64_t num_walks, int32_t walk_length, const void* n_out,
               const void* e_out, int32_t out_type, const void* work, size_t work_bytes) {
    if (int rc = check_graph(rowptr, num_nodes, col, num_edges, start, num_walks, walk_length,
                             n_out))
        return rc;
    if (int rc = check_out_type(out_type, num_nodes, num_edges, e_out)) return rc;
    return check_workspace(work, work_bytes);
}

// first_walk of the seeded entry points: the Philox stream index of walk 0,
// with every stream position (first_walk + num_walks) * walk_length in int64.
int check_first_walk(int64_t first_walk, int64_t num_walks, int32_t walk_length) {
    if (first_walk < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "first_walk must be >= 0");
    const int64_t per = walk_length > 0 ? walk_length : 1;
    if (first_walk > INT64_MAX / per - num_walks)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "(first_walk + num_walks) * walk_length overflows int64");
    return MLXC_OK;
}

// Parameters of one node2vec call; the acceptance constants exactly as
// BiasedRandomWalk.cpp:52-55, in FP64.
int n2v_params(double p, double q, uint64_t seed, int32_t rule, int32_t rows, N2VParams& prm) {
    if (!(p > 0.0) || !(q > 0.0) || !std::isfinite(p) || !std::isfinite(q))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "p and q must be finite and > 0");
    if (rule != MLXC_RULE_REF_CHAIN && rule != MLXC_RULE_NODE2VEC_EXACT)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "rule must be MLXC_RULE_REF_CHAIN or MLXC_RULE_NODE2VEC_EXACT");
    const int32_t order = rows & ~MLXC_ROWS_SYMMETRIC;
    if (order != MLXC_ROWS_UNSORTED && order != MLXC_ROWS_SORTED && order != MLXC_ROWS_DETECT)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "rows must be MLXC_ROWS_UNSORTED, MLXC_ROWS_SORTED or MLXC_ROWS_DETECT, "
                    "optionally with MLXC_ROWS_SYMMETRIC");
    const double max_prob = std::fmax(std::fmax(1. / p, 1.), 1. / q);
    prm.prob0 = 1. / p / max_prob;
    prm.prob1 = 1. / max_prob;
    prm.prob2 = 1. / q / max_prob;
    prm.key0 = static_cast<uint32_t>(seed);
    prm.key1 = static_cast<uint32_t>(seed >> 32);
    prm.rule = rule;
    prm.rows = order;
    prm.symmetric = (rows & MLXC_ROWS_SYMMETRIC) != 0;
    prm.out_type = MLXC_OUT_INT64;
    return MLXC_OK;
}

// Arguments of mlxc_csr_build and its host twin.
int check_csr_build(const int64_t* row, const int64_t* col, int64_t num_edges, int64_t num_nodes,
                    int32_t flags, const int64_t* rowptr, const int64_t* col_out) {
    if (num_edges < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_edges must be >= 0");
    if (num_nodes < 0 || num_nodes > (int64_t(1) << 32))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes must lie in [0, 2^32]");
    if (flags & ~(MLXC_CSR_SYMMETRIZE | MLXC_CSR_DEDUP))
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "flags must be a combination of MLXC_CSR_SYMMETRIZE and MLXC_CSR_DEDUP");
    if (num_edges > (INT64_MAX / 64))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "num_edges too large");
    if (!rowptr) return fail(MLXC_ERR_INVALID_ARGUMENT, "rowptr must not be NULL");
    if (num_edges > 0 && (!row || !col || !col_out))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "row, col and col_out must not be NULL");
    return MLXC_OK;
}

int check_windows(const void* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                  int32_t elem_type, const void* out) {
    if (num_walks < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "num_walks must be >= 0");
    if (elem_type != MLXC_OUT_INT64 && elem_type != MLXC_OUT_INT32)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "element type must be MLXC_OUT_INT64 or MLXC_OUT_INT32");
    if (walk_nodes < 1 || walk_nodes > windows_max_nodes(elem_type))
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "nodes per walk must lie in [1, 65536 / element size]");
    if (ctx < 1 || ctx > 32 || ctx > walk_nodes)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "context_size must lie in [1, min(32, nodes per walk)]");
    if (num_walks > 0 && (!walks || !out))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "walks and out must not be NULL");
    if (num_walks > INT64_MAX / 32 / walk_nodes)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "output size overflows int64");
    return MLXC_OK;
}

// The window kernels launch one block of kBlock threads per tile of walks,
// and a launch holds fewer than 2^32 work-items per grid dimension.
int check_window_grid(int64_t num_walks, int32_t walk_nodes, int32_t elem_type) {
    const int per_block = tile_walks(walk_nodes, elem_type == MLXC_OUT_INT32 ? 4 : 8);
    const int64_t max_blocks = static_cast<int64_t>(UINT32_MAX) / kBlock;
    if (per_block >= 1 && (num_walks + per_block - 1) / per_block > max_blocks)
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "too many walks for one window launch: at most " +
                        std::to_string(max_blocks * per_block) +
                        " walks of this length; split the call");
    return MLXC_OK;
}

int check_negative(const int64_t* start, int64_t num_walks, int32_t walk_length, int32_t ctx,
                   int64_t num_nodes, int32_t out_type, const void* out) {
    if (int rc = check_walk_length(walk_length)) return rc;
    if (int rc = check_windows(start, num_walks, walk_length + 1, ctx, out_type, out)) return rc;
    if (num_nodes < 1 || num_nodes > (int64_t(1) << 32))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes must lie in [1, 2^32]");
    if (out_type == MLXC_OUT_INT32 && num_nodes > INT32_MAX)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "MLXC_OUT_INT32 needs num_nodes below 2^31");
    return MLXC_OK;
}

// Device address of the current device's scratch array, looked up with
// that device current on the first call there and kept per device.
int noalloc_scratch(void** out) {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    MLXC_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(MLXC_ERR_HIP, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        MLXC_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(MLXC_ERR_HIP, "hipGetSymbolAddress returned NULL for the scratch array");
        addr[dev] = p;
    }
    *out = addr[dev];
    return MLXC_OK;
}

HostWalk host_walk(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                   int64_t num_edges, const int64_t* start, int64_t num_walks, const float* rand,
                   int32_t walk_length, uint64_t seed, int64_t first_walk, void* n_out,
                   void* e_out, int32_t out_type) {
    return HostWalk{rowptr, col, start, rand, n_out, e_out, out_type, num_nodes, num_edges,
                    num_walks, walk_length, static_cast<uint32_t>(seed),
                    static_cast<uint32_t>(seed >> 32), first_walk};
}

// The status word of a call (workspace word 0) into host memory, then the
// flag that it is there: system-scope stores, the flag's with release order.
__global__ void publish_status_kernel(const int64_t* work, int64_t* h_status) {
    if (threadIdx.x == 0) {
        const int64_t bits = work[0];
        __hip_atomic_store(h_status + 1, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(h_status, int64_t{1}, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace
}  // namespace mlxc

using namespace mlxc;

extern "C" {

int mlxc_version(void) { return 301; }

const char* mlxc_last_error(void) { return g_last_error.c_str(); }

int mlxc_publish_status(const void* d_workspace, int64_t* h_status, void* stream) {
    if (int rc = check_workspace(d_workspace, MLXC_WORK_WORDS * sizeof(int64_t))) return rc;
    if (!h_status || reinterpret_cast<uintptr_t>(h_status) % 8 != 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "h_status must be 8-byte aligned host memory");
    int64_t* d_status = nullptr;  // the device's address of the host words
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&d_status), h_status, 0) != hipSuccess) {
        (void)hipGetLastError();  // not left for the next call's launch check
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "h_status is not host memory the device can write (hipHostMalloc)");
    }
    hipLaunchKernelGGL(publish_status_kernel, dim3(1), dim3(kWave), 0,
                       static_cast<hipStream_t>(stream), static_cast<const int64_t*>(d_workspace),
                       d_status);
    MLXC_HIP_TRY(hipGetLastError());
    return MLXC_OK;
}

int mlxc_set_walk_events(void* start_event, void* stop_event) {
    if ((start_event == nullptr) != (stop_event == nullptr))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "set both events or neither");
    g_walk_events[0] = static_cast<hipEvent_t>(start_event);
    g_walk_events[1] = static_cast<hipEvent_t>(stop_event);
    return MLXC_OK;
}

size_t mlxc_random_walk_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                                        int32_t walk_length) {
    return uniform_workspace_bytes(num_nodes, num_edges, num_walks, walk_length);
}

size_t mlxc_rejection_sampling_workspace_bytes(int64_t num_nodes, int64_t num_edges,
                                               int64_t num_walks, int32_t walk_length, double p,
                                               double q, int32_t rule) {
    N2VParams prm;
    // invalid parameters: the call will fail; any size will do
    const double width = n2v_params(p, q, 0, rule, MLXC_ROWS_DETECT, prm) == MLXC_OK
                             ? n2v_search_width(prm)
                             : 1.0;
    return node2vec_workspace_bytes(num_nodes, num_edges, num_walks, walk_length, width);
}

size_t mlxc_rejection_sampling_layout_bytes(int64_t num_nodes, int64_t num_edges,
                                            int64_t num_walks, int32_t walk_length,
                                            int32_t layout) {
    return node2vec_layout_bytes(num_nodes, num_edges, num_walks, walk_length, layout);
}

int mlxc_random_walk(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                     int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                     const float* d_rand, int32_t walk_length, void* d_n_out, void* d_e_out,
                     int32_t out_type, void* d_workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_walk(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                            walk_length, d_n_out, d_e_out, out_type, d_workspace, workspace_bytes))
        return rc;
    if (num_walks > 0 && walk_length > 0 && !d_rand)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "rand must not be NULL");
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (num_walks == 0) return launch_zero_work(d_work, s);  // (else the walk's launches zero it)
    const WalkArgs a{d_rowptr, d_col, d_start, d_rand, d_n_out, d_e_out, d_work,
                     num_nodes, num_edges, num_walks, walk_length, 0u, 0u, 0};
    return launch_uniform(a, d_workspace, workspace_bytes, false, out_type, s);
}

int mlxc_random_walk_noalloc(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                             int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                             const float* d_rand, int32_t walk_length, void* d_n_out,
                             void* d_e_out, int32_t out_type, int64_t* d_status, void* stream) {
    if (int rc = check_graph(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                             walk_length, d_n_out))
        return rc;
    if (int rc = check_out_type(out_type, num_nodes, num_edges, d_e_out)) return rc;
    if (num_walks > 0 && walk_length > 0 && !d_rand)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "rand must not be NULL");
    // the queried size, or the whole array when the fastest layout needs more:
    // the walk then runs the largest layout the array holds (start records
    // only, or none), with the same results
    size_t need = uniform_workspace_bytes(num_nodes, num_edges, num_walks, walk_length);
    if (need > static_cast<size_t>(MLXC_NOALLOC_SCRATCH_BYTES)) need = MLXC_NOALLOC_SCRATCH_BYTES;
    void* ws = nullptr;
    if (int rc = noalloc_scratch(&ws)) return rc;
    // the same call as mlxc_random_walk with a workspace of that size; its
    // launches clear the status words first, so stale contents of the shared
    // array do not matter
    if (int rc = mlxc_random_walk(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                                  d_rand, walk_length, d_n_out, d_e_out, out_type, ws, need,
                                  stream))
        return rc;
    if (!d_status) return MLXC_OK;
    return launch_copy_word(static_cast<const int64_t*>(ws), d_status,
                            static_cast<hipStream_t>(stream));
}

int mlxc_random_walk_seeded(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                            int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                            int32_t walk_length, uint64_t seed, int64_t first_walk,
                            void* d_n_out, void* d_e_out, int32_t out_type, void* d_workspace,
                            size_t workspace_bytes, void* stream) {
    if (int rc = check_walk(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                            walk_length, d_n_out, d_e_out, out_type, d_workspace, workspace_bytes))
        return rc;
    if (int rc = check_first_walk(first_walk, num_walks, walk_length)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (num_walks == 0) return launch_zero_work(d_work, s);  // (else the walk's launches zero it)
    const WalkArgs a{d_rowptr, d_col, d_start, nullptr, d_n_out, d_e_out, d_work,
                     num_nodes, num_edges, num_walks, walk_length,
                     static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32), first_walk};
    return launch_uniform(a, d_workspace, workspace_bytes, true, out_type, s);
}

int mlxc_rejection_sampling(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                            int64_t num_edges, const int64_t* d_start, int64_t num_walks,
                            int32_t walk_length, double p, double q, uint64_t seed,
                            int64_t first_walk, int32_t rule, int32_t rows, void* d_n_out,
                            void* d_e_out, int32_t out_type, void* d_workspace,
                            size_t workspace_bytes, void* stream) {
    if (int rc = check_walk(d_rowptr, num_nodes, d_col, num_edges, d_start, num_walks,
                            walk_length, d_n_out, d_e_out, out_type, d_workspace, workspace_bytes))
        return rc;
    if (int rc = check_first_walk(first_walk, num_walks, walk_length)) return rc;
    N2VParams prm;
    if (int rc = n2v_params(p, q, seed, rule, rows, prm)) return rc;
    prm.out_type = out_type;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (int rc = launch_zero_work(d_work, s)) return rc;
    if (num_walks == 0) return MLXC_OK;
    const WalkArgs a{d_rowptr, d_col, d_start, nullptr, d_n_out, d_e_out, d_work,
                     num_nodes, num_edges, num_walks, walk_length, 0u, 0u, first_walk};
    return launch_node2vec(a, prm, d_workspace, workspace_bytes, s);
}

int mlxc_csr_check(const int64_t* d_rowptr, int64_t num_nodes, const int64_t* d_col,
                   int64_t num_edges, void* d_workspace, size_t workspace_bytes, int32_t* h_flags,
                   void* stream) {
    if (num_nodes < 0 || num_edges < 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "num_nodes and num_edges must be >= 0");
    if (!d_rowptr || !h_flags || (num_edges > 0 && !d_col))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "NULL pointer argument");
    if (int rc = check_workspace(d_workspace, workspace_bytes)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t* d_work = static_cast<int64_t*>(d_workspace);
    if (int rc = launch_zero_work(d_work, s)) return rc;
    if (int rc = launch_csr_check(d_rowptr, num_nodes, d_col, num_edges, d_work, s)) return rc;
    if (int rc = launch_csr_symmetry(d_rowptr, num_nodes, d_col, num_edges, d_work, s)) return rc;
    int64_t host[4] = {0, 0, 0, 0};
    MLXC_HIP_TRY(hipMemcpyAsync(host, d_work, sizeof(host), hipMemcpyDeviceToHost, s));
    MLXC_HIP_TRY(hipStreamSynchronize(s));
    int32_t flags = static_cast<int32_t>(host[0]);
    if (!(flags & MLXC_CSR_BAD_ROWPTR) && host[1] != host[2]) flags |= MLXC_CSR_UNSORTED;
    if (host[3]) flags |= MLXC_CSR_ASYMMETRIC;
    *h_flags = flags;
    return MLXC_OK;
}

int mlxc_philox_uniform(float* d_out, int64_t n, uint64_t seed, void* stream) {
    if (n < 0) return fail(MLXC_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n == 0) return MLXC_OK;
    if (!d_out) return fail(MLXC_ERR_INVALID_ARGUMENT, "out must not be NULL");
    return launch_philox_fill(d_out, n, seed, static_cast<hipStream_t>(stream));
}

size_t mlxc_csr_build_workspace_bytes(int64_t num_nodes, int64_t num_edges, int32_t flags) {
    if (num_nodes < 0 || num_edges < 0 || num_edges > INT64_MAX / 64) return 0;
    return csr_build_workspace_bytes(num_nodes, num_edges, flags);
}

int mlxc_csr_build(const int64_t* d_row, const int64_t* d_col, int64_t num_edges,
                   int64_t num_nodes, int32_t flags, int64_t* d_rowptr, int64_t* d_col_out,
                   void* d_workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_csr_build(d_row, d_col, num_edges, num_nodes, flags, d_rowptr, d_col_out))
        return rc;
    if (int rc = check_workspace(d_workspace, workspace_bytes)) return rc;
    return launch_csr_build(d_row, d_col, num_edges, num_nodes, flags, d_rowptr, d_col_out,
                            d_workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int mlxc_csr_build_cpu(const int64_t* row, const int64_t* col, int64_t num_edges,
                       int64_t num_nodes, int32_t flags, int64_t* rowptr, int64_t* col_out,
                       int64_t* count, int64_t* status) {
    if (int rc = check_csr_build(row, col, num_edges, num_nodes, flags, rowptr, col_out))
        return rc;
    if (!count) return fail(MLXC_ERR_INVALID_ARGUMENT, "count must not be NULL");
    uint32_t bits = 0;
    int64_t n = 0;
    const int rc = host_csr_build(row, col, num_edges, num_nodes, flags, rowptr, col_out, n, bits);
    *count = n;
    if (status) *status = bits;
    return rc;
}

int mlxc_context_windows(const void* d_walks, int64_t num_walks, int32_t walk_nodes,
                         int32_t context_size, int32_t elem_type, void* d_out, void* stream) {
    if (int rc = check_windows(d_walks, num_walks, walk_nodes, context_size, elem_type, d_out))
        return rc;
    if (int rc = check_window_grid(num_walks, walk_nodes, elem_type)) return rc;
    if (num_walks == 0) return MLXC_OK;
    return launch_context_windows(d_walks, num_walks, walk_nodes, context_size, elem_type, d_out,
                                  static_cast<hipStream_t>(stream));
}

int mlxc_negative_windows(const int64_t* d_start, int64_t num_walks, int32_t walk_length,
                          int32_t context_size, int64_t num_nodes, uint64_t seed,
                          int32_t out_type, void* d_out, void* stream) {
    if (int rc = check_negative(d_start, num_walks, walk_length, context_size, num_nodes,
                                out_type, d_out))
        return rc;
    if (int rc = check_window_grid(num_walks, walk_length + 1, out_type)) return rc;
    if (num_walks == 0) return MLXC_OK;
    return launch_negative_windows(d_start, num_walks, walk_length, context_size, num_nodes, seed,
                                   out_type, d_out, static_cast<hipStream_t>(stream));
}

int mlxc_gather_probe(const void* d_table, int64_t table_bytes, int32_t load_bytes,
                      int32_t loads_per_lane, int32_t dependent, int32_t blocks_per_cu,
                      int64_t iterations, uint64_t seed, uint32_t* d_sink,
                      int64_t* loads_issued, void* stream) {
    if (!d_table || !d_sink || !loads_issued)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "table, sink and loads_issued must not be NULL");
    if (reinterpret_cast<uintptr_t>(d_table) % 16 != 0)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "table must be 16-byte aligned");
    if (load_bytes != 4 && load_bytes != 16)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "load_bytes must be 4 or 16");
    if (table_bytes < load_bytes || table_bytes / load_bytes > int64_t{UINT32_MAX})
        return fail(MLXC_ERR_INVALID_ARGUMENT,
                    "table_bytes must lie in [load_bytes, load_bytes * (2^32 - 1)]");
    if (loads_per_lane != 1 && loads_per_lane != 2 && loads_per_lane != 4 && loads_per_lane != 8)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "loads_per_lane must be 1, 2, 4 or 8");
    if (dependent != 0 && dependent != 1)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "dependent must be 0 or 1");
    if (blocks_per_cu < 1 || blocks_per_cu > 32)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "blocks_per_cu must lie in [1, 32]");
    if (iterations < 1 || iterations > (int64_t{1} << 24))
        return fail(MLXC_ERR_INVALID_ARGUMENT, "iterations must lie in [1, 2^24]");
    return launch_gather_probe(d_table, table_bytes, load_bytes, loads_per_lane, dependent,
                               blocks_per_cu, iterations, seed, d_sink, loads_issued,
                               static_cast<hipStream_t>(stream));
}

int mlxc_context_windows_cpu(const void* walks, int64_t num_walks, int32_t walk_nodes,
                             int32_t context_size, int32_t elem_type, void* out) {
    if (int rc = check_windows(walks, num_walks, walk_nodes, context_size, elem_type, out))
        return rc;
    host_context_windows(walks, num_walks, walk_nodes, context_size, elem_type, out);
    return MLXC_OK;
}

int mlxc_negative_windows_cpu(const int64_t* start, int64_t num_walks, int32_t walk_length,
                              int32_t context_size, int64_t num_nodes, uint64_t seed,
                              int32_t out_type, void* out) {
    if (int rc = check_negative(start, num_walks, walk_length, context_size, num_nodes, out_type,
                                out))
        return rc;
    host_negative_windows(start, num_walks, walk_length, context_size, num_nodes, seed, out_type,
                          out);
    return MLXC_OK;
}

int mlxc_random_walk_cpu(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                         int64_t num_edges, const int64_t* start, int64_t num_walks,
                         const float* rand, int32_t walk_length, void* n_out, void* e_out,
                         int32_t out_type, int32_t threads, int64_t* status) {
    if (int rc = check_graph(rowptr, num_nodes, col, num_edges, start, num_walks, walk_length,
                             n_out))
        return rc;
    if (int rc = check_out_type(out_type, num_nodes, num_edges, e_out)) return rc;
    if (num_walks > 0 && walk_length > 0 && !rand)
        return fail(MLXC_ERR_INVALID_ARGUMENT, "rand must not be NULL");
    uint32_t bits = 0;
    const HostWalk w = host_walk(rowptr, num_nodes, col, num_edges, start, num_walks, rand,
                                 walk_length, 0, 0, n_out, e_out, out_type);
    const int rc = host_uniform(w, false, threads, bits);
    if (status) *status = bits;
    return rc;
}

int mlxc_random_walk_seeded_cpu(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                                int64_t num_edges, const int64_t* start, int64_t num_walks,
                                int32_t walk_length, uint64_t seed, int64_t first_walk,
                                void* n_out, void* e_out, int32_t out_type, int32_t threads,
                                int64_t* status) {
    if (int rc = check_graph(rowptr, num_nodes, col, num_edges, start, num_walks, walk_length,
                             n_out))
        return rc;
    if (int rc = check_out_type(out_type, num_nodes, num_edges, e_out)) return rc;
    if (int rc = check_first_walk(first_walk, num_walks, walk_length)) return rc;
    uint32_t bits = 0;
    const HostWalk w = host_walk(rowptr, num_nodes, col, num_edges, start, num_walks, nullptr,
                                 walk_length, seed, first_walk, n_out, e_out, out_type);
    const int rc = host_uniform(w, true, threads, bits);
    if (status) *status = bits;
    return rc;
}

int mlxc_rejection_sampling_cpu(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                                int64_t num_edges, const int64_t* start, int64_t num_walks,
                                int32_t walk_length, double p, double q, uint64_t seed,
                                int64_t first_walk, int32_t rule, int32_t rows, void* n_out,
                                void* e_out, int32_t out_type, int32_t threads,
                                int64_t* status) {
    if (int rc = check_graph(rowptr, num_nodes, col, num_edges, start, num_walks, walk_length,
                             n_out))
        return rc;
    if (int rc = check_out_type(out_type, num_nodes, num_edges, e_out)) return rc;
    if (int rc = check_first_walk(first_walk, num_walks, walk_length)) return rc;
    N2VParams prm;
    if (int rc = n2v_params(p, q, seed, rule, rows, prm)) return rc;
    prm.out_type = out_type;
    uint32_t bits = 0;
    const HostWalk w = host_walk(rowptr, num_nodes, col, num_edges, start, num_walks, nullptr,
                                 walk_length, seed, first_walk, n_out, e_out, out_type);
    const int rc = host_node2vec(w, prm, threads, bits);
    if (status) *status = bits;
    return rc;
}

}  // extern "C"
