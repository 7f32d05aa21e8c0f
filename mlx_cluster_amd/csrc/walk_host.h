// Host-side internals shared by the translation units of libmlxc.so: error
// reporting, device properties, grid sizing and the launchers each file
// provides.  Nothing here is part of the C ABI (include/mlxc.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "mlxc.h"
#include "walk_device.h"

namespace mlxc {

// Records msg as the calling thread's last error and returns code.
int fail(int code, const std::string& msg);

#define MLXC_HIP_TRY(expr)                                                                   \
    do {                                                                                     \
        hipError_t err_ = (expr);                                                            \
        if (err_ != hipSuccess)                                                              \
            return ::mlxc::fail(MLXC_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(err_)); \
    } while (0)

// The events the calling thread set with mlxc_set_walk_events (null: none),
// recorded on a call's stream right before (0) and right after (1) its walk
// kernel, the last launch of the call.
extern thread_local hipEvent_t g_walk_events[2];

inline int record_walk_event(int which, hipStream_t stream) {
    if (g_walk_events[which]) MLXC_HIP_TRY(hipEventRecord(g_walk_events[which], stream));
    return MLXC_OK;
}

struct DeviceInfo {
    int cus = 0;  // compute units of the current device
};

// Properties of the current device (cached per device).
int device_info(DeviceInfo& info);

// Grid for a grid-stride kernel over `items`: enough blocks to cover them,
// at most blocks_per_cu per compute unit.
int stream_grid(int64_t items, int blocks_per_cu, int& grid);

// Persistent grid: the blocks that stay resident on the device (at most
// max_per_cu per compute unit when max_per_cu > 0), but no more than the
// walks can feed (each block serves slots * kBlock walks at once).
template <typename Kernel>
int persistent_grid(Kernel kernel, int64_t num_walks, int slots, int& grid, int max_per_cu = 0) {
    DeviceInfo info;
    if (int rc = device_info(info)) return rc;
    int per_cu = 0;
    MLXC_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kBlock, 0));
    if (max_per_cu > 0 && per_cu > max_per_cu) per_cu = max_per_cu;
    if (per_cu < 1) per_cu = 1;
    const int64_t resident = static_cast<int64_t>(info.cus) * per_cu;
    const int64_t per_block = static_cast<int64_t>(slots) * kBlock;
    const int64_t feedable = (num_walks + per_block - 1) / per_block;
    grid = static_cast<int>(feedable < resident ? feedable : resident);
    if (grid < 1) grid = 1;
    return MLXC_OK;
}

// Graphs small enough that building their edge records (one parallel pass,
// about E / 3e10 s) costs less than the dependent read per step it saves on
// the walk's serial chain (about 1 us per step when few walks run): records
// then pay off whatever the number of walks.
constexpr int64_t kSmallGraphEdgesPerStep = 32768;

// Node ids and edge offsets fit the int32 fields of the record layouts.
inline bool records_fit(int64_t num_nodes, int64_t num_edges) {
    return num_nodes <= INT32_MAX && num_edges <= INT32_MAX;
}

// ---- prep_kernels.hip
int launch_zero_work(int64_t* d_work, hipStream_t stream);
// The uniform record walk's preparation in one launch: zeroes the status
// words, writes the edge records and, after them, the start records; in the
// 8-byte format *packed when packed is not null, else as EdgeRecord.
int launch_record_prep(const int64_t* rowptr, const int64_t* col, const int64_t* start,
                       int64_t num_nodes, int64_t num_edges, int64_t num_walks, void* recs,
                       const PackedFormat* packed, int64_t* work, hipStream_t stream);
// Edge records and the search index levels (index.count > 0) of the node2vec
// walk, and in the same pass the start records of `starts` (num_walks 0:
// none); a non-null check_work also validates the CSR and counts row
// descents (see edge_record_kernel).
// A non-null row32 (num_nodes + 1 int32 of workspace) makes the pass first
// convert rowptr to int32 row starts and gather the rows from them.
int launch_edge_records(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                        int64_t num_edges, EdgeRecord* recs, const IndexLevels& index,
                        const StartRecords& starts, int64_t* check_work, hipStream_t stream,
                        const HubBitmaps& hubs, int32_t* row32);
// The hub bitmaps (see HubBitmaps), in two launches around
// launch_edge_records: launch_hub_bitmaps chooses the degree threshold (at
// least min_degree) and assigns the slots, which the records then carry;
// launch_hub_build, after the records (whose pass counts the row descents
// that tell it whether rows are sorted), fills the bitmaps.  Nothing when
// hubs.max == 0.
int launch_hub_bitmaps(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                       int64_t num_edges, const HubBitmaps& hubs, int64_t min_degree,
                       hipStream_t stream);
int launch_hub_build(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                     const HubBitmaps& hubs, int32_t rows, const int64_t* work,
                     hipStream_t stream);
// The row hash tables (see row_hashed) from the int32 row starts and col32,
// after launch_edge_records wrote both; hub_info (null: no hub bitmaps in
// this call) gives the hub threshold, above which rows get no table.
// long_rows (num_nodes int32) and *long_count: scratch of the build.
int launch_hash_build(const int32_t* row32, const int32_t* col32, int64_t num_nodes,
                      const int64_t* hub_info, int32_t* table, int32_t* long_rows,
                      int64_t* long_count, hipStream_t stream);
// The index levels alone, from col (node2vec CSR mode), and the start records;
// a 16-byte aligned col uses four entries per thread, any other alignment the
// record pass.
int launch_edge_index(const int64_t* rowptr, const int64_t* col, int64_t num_nodes,
                      int64_t num_edges, const IndexLevels& index, const StartRecords& starts,
                      int64_t* check_work, hipStream_t stream, int32_t* row32);
// Start records of the uniform CSR walk; the same launch zeroes the call's
// status words.
int launch_walk_init(const int64_t* rowptr, const int64_t* start, int64_t num_nodes,
                     int64_t num_edges, int64_t num_walks, EdgeRecord* init, int64_t* work,
                     hipStream_t stream);
// work[0] |= MLXC_CSR_* bits, work[1] += the row descents that start no row
// (rows sorted iff work[1] == work[2], which stays 0); the words must start
// at zero.
int launch_csr_check(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                     int64_t num_edges, int64_t* d_work, hipStream_t stream);
// After launch_csr_check, on a well-formed graph with sorted rows: work[3] = 1
// when some entry (u, v) has no reverse (v, u).
int launch_csr_symmetry(const int64_t* rowptr, int64_t num_nodes, const int64_t* col,
                        int64_t num_edges, int64_t* d_work, hipStream_t stream);
// Turns the words of launch_csr_check into a walk's: status bits in work[0],
// work[1] = 0, work[2] = 1 if every row is sorted, work[3] = 0.
int launch_csr_status(int64_t* d_work, hipStream_t stream);
// *d_dst = *d_src on the stream (a kernel, so the call can be captured).
int launch_copy_word(const int64_t* d_src, int64_t* d_dst, hipStream_t stream);
int launch_philox_fill(float* out, int64_t n, uint64_t seed, hipStream_t stream);

// ---- uniform_walk.hip
size_t uniform_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                               int32_t walk_length);
// generate: the kernels compute their uniforms from the Philox key in a
// (key0, key1) instead of reading a.rand.  out_type: MLXC_OUT_* of a.n_out
// and a.e_out.
int launch_uniform(const WalkArgs& a, void* workspace, size_t workspace_bytes, bool generate,
                   int32_t out_type, hipStream_t stream);

// ---- node2vec_walk.hip
struct N2VParams {
    double prob0, prob1, prob2;  // acceptance constants, BiasedRandomWalk.cpp:52-55
    uint32_t key0, key1;         // Philox key (the seed)
    int32_t rule;                // MLXC_RULE_*
    int32_t rows;                // MLXC_ROWS_UNSORTED / SORTED / DETECT
    int32_t symmetric;           // MLXC_ROWS_SYMMETRIC was given
    int32_t out_type;            // MLXC_OUT_*
};
// Share of acceptance draws r for which a trial may need the row search.
double n2v_search_width(const N2VParams& p);
size_t node2vec_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                                int32_t walk_length, double search_width);
// Bytes of one MLXC_N2V_LAYOUT_* layout (0: not available for this call).
size_t node2vec_layout_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                             int32_t walk_length, int32_t layout);
int launch_node2vec(const WalkArgs& a, const N2VParams& p, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);

// ---- csr_build.hip
size_t csr_build_workspace_bytes(int64_t num_nodes, int64_t num_edges, int32_t flags);
int launch_csr_build(const int64_t* row, const int64_t* col, int64_t num_edges, int64_t num_nodes,
                     int32_t flags, int64_t* rowptr, int64_t* col_out, void* workspace,
                     size_t workspace_bytes, hipStream_t stream);

// ---- windows.hip
int launch_context_windows(const void* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                           int32_t elem_type, void* out, hipStream_t stream);
int launch_negative_windows(const int64_t* start, int64_t num_walks, int32_t walk_length,
                            int32_t ctx, int64_t num_nodes, uint64_t seed, int32_t out_type,
                            void* out, hipStream_t stream);
// Most nodes per walk the window kernels accept for this element type (a
// walk row must fit the LDS tile).
int windows_max_nodes(int32_t elem_type);
// Walks per block of the window kernels (one block per tile of walks).
int tile_walks(int32_t walk_nodes, size_t esz);

// ---- gather_probe.hip
// Random reads from a device table (mlxc_gather_probe; arguments checked by
// the caller); *loads_issued receives the number of loads the launch makes.
int launch_gather_probe(const void* table, int64_t table_bytes, int32_t load_bytes,
                        int32_t loads_per_lane, int32_t dependent, int32_t blocks_per_cu,
                        int64_t iterations, uint64_t seed, uint32_t* sink, int64_t* loads_issued,
                        hipStream_t stream);

// ---- host_walk.cpp (host pointers; the same walks on CPU threads)
struct HostWalk {
    const int64_t* rowptr;
    const int64_t* col;
    const int64_t* start;
    const float* rand;  // null when the uniforms are generated
    void* n_out;        // int64 or int32 (out_type)
    void* e_out;        // may be null
    int32_t out_type;   // MLXC_OUT_*
    int64_t num_nodes, num_edges, num_walks, walk_length;
    uint32_t key0, key1;  // Philox key of generated uniforms
    int64_t walk_base;    // Philox stream index of walk 0 (WalkArgs::walk_base)
};
// threads <= 0: one per hardware thread.  status receives MLXC_STATUS_* bits.
int host_uniform(const HostWalk& w, bool generate, int32_t threads, uint32_t& status);
int host_node2vec(const HostWalk& w, const N2VParams& p, int32_t threads, uint32_t& status);
// The windows of mlxc_context_windows / mlxc_negative_windows from host arrays.
void host_context_windows(const void* walks, int64_t num_walks, int32_t walk_nodes, int32_t ctx,
                          int32_t elem_type, void* out);
void host_negative_windows(const int64_t* start, int64_t num_walks, int32_t walk_length,
                           int32_t ctx, int64_t num_nodes, uint64_t seed, int32_t out_type,
                           void* out);
// The CSR of mlxc_csr_build from host arrays.
int host_csr_build(const int64_t* row, const int64_t* col, int64_t num_edges, int64_t num_nodes,
                   int32_t flags, int64_t* rowptr, int64_t* col_out, int64_t& count,
                   uint32_t& status);

}  // namespace mlxc
