// Host twin of mlxc_csr_build (csr_build.hip): the same CSR from host arrays.
// Keys are packed, clamped and ordered exactly as on the device, so the two
// agree entry for entry, malformed input included.
#include <algorithm>
#include <vector>

#include "walk_host.h"

namespace mlxc {

int host_csr_build(const int64_t* row, const int64_t* col, int64_t num_edges, int64_t num_nodes,
                   int32_t flags, int64_t* rowptr, int64_t* col_out, int64_t& count,
                   uint32_t& status) {
    const int64_t total = (flags & MLXC_CSR_SYMMETRIZE) ? 2 * num_edges : num_edges;
    int cbits = 0;
    for (uint64_t x = num_nodes > 1 ? static_cast<uint64_t>(num_nodes - 1) : 0; x; x >>= 1)
        ++cbits;
    std::vector<uint64_t> keys(static_cast<size_t>(total));
    for (int64_t i = 0; i < total; ++i) {
        int64_t r, c;
        if (i < num_edges) {
            r = row[i];
            c = col[i];
        } else {
            r = col[i - num_edges];
            c = row[i - num_edges];
        }
        // an id outside [0, num_nodes) becomes 0, each on its own
        if (static_cast<uint64_t>(r) >= static_cast<uint64_t>(num_nodes)) {
            status |= MLXC_STATUS_BAD_NODE;
            r = 0;
        }
        if (static_cast<uint64_t>(c) >= static_cast<uint64_t>(num_nodes)) {
            status |= MLXC_STATUS_BAD_NODE;
            c = 0;
        }
        keys[i] = (static_cast<uint64_t>(r) << cbits) | static_cast<uint64_t>(c);
    }
    std::sort(keys.begin(), keys.end());
    if (flags & MLXC_CSR_DEDUP) keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
    const uint64_t cmask = cbits == 0 ? 0 : (~uint64_t(0) >> (64 - cbits));
    std::fill(rowptr, rowptr + num_nodes + 1, int64_t(0));
    const int64_t n = static_cast<int64_t>(keys.size());
    for (int64_t i = 0; i < n; ++i) {
        col_out[i] = static_cast<int64_t>(keys[i] & cmask);
        ++rowptr[static_cast<int64_t>(keys[i] >> cbits) + 1];
    }
    for (int64_t v = 0; v < num_nodes; ++v) rowptr[v + 1] += rowptr[v];
    count = n;
    return MLXC_OK;
}

}  // namespace mlxc
