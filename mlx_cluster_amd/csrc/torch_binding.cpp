// Compiled fast path of the Python surface for the common call: every array a
// torch tensor of the right dtype, contiguous, on the current device, the
// call on torch's current stream.  It does what walks.py does for such calls
// (check the arguments, allocate the outputs and workspace from torch's
// caching allocator, launch through the C ABI, read the status word) without
// the Python layer's per-call cost, which bounds the reference tests' own
// calls (2,000 walks of 5 steps on a Cora-sized graph).  Any other call
// returns None and walks.py takes it.  Errors raise as in walks.py.
//
// Mirrors: random_walk / rejection_sampling of /root/reference/bindings.cpp:12-63.
#include <ATen/hip/HIPContext.h>
#include <hip/hip_runtime.h>
#include <pybind11/pybind11.h>
#include <torch/extension.h>

#include <chrono>
#include <optional>
#include <string>

#include "mlxc.h"

namespace py = pybind11;

namespace {

// Whether t can be passed as is: a contiguous tensor of dtype on device.
bool usable(const at::Tensor& t, at::ScalarType dtype, const at::Device& device) {
    return t.scalar_type() == dtype && t.device() == device && t.is_contiguous();
}

const void* data_or_null(const at::Tensor& t) { return t.numel() ? t.data_ptr() : nullptr; }

void raise_code(int rc, const char* what) {
    const std::string msg = std::string(what) + ": " + mlxc_last_error();
    if (rc == MLXC_ERR_INVALID_ARGUMENT) throw py::value_error(msg);
    throw std::runtime_error(msg);
}

// The calling thread's two host words for mlxc_publish_status: allocated at
// the thread's first validated call (one pinned page) and kept for the rest
// of the process, since freeing them at thread exit could run after the HIP
// runtime has shut down; null if the allocation failed.
int64_t* status_words() {
    thread_local int64_t* words = [] {
        void* p = nullptr;
        if (hipHostMalloc(&p, 2 * sizeof(int64_t),
                          hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable) !=
            hipSuccess) {
            (void)hipGetLastError();
            return static_cast<int64_t*>(nullptr);
        }
        return static_cast<int64_t*>(p);
    }();
    return words;
}

// The status word of the call just enqueued on `stream`.  The device stores
// it into this thread's host words (mlxc_publish_status) and the host waits
// for the flag: spinning for up to about 200 us (the reference tests' calls
// take tens), then in hipStreamSynchronize.  Without the host words, torch's
// scalar read (a copy ordered on the stream, about 13 us more per call).
int64_t read_status(const at::Tensor& work, hipStream_t stream) {
    int64_t* h = status_words();
    if (h) {
        __atomic_store_n(&h[0], int64_t{0}, __ATOMIC_RELAXED);
        if (mlxc_publish_status(work.data_ptr(), h, stream) == MLXC_OK) {
            const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(200);
            for (unsigned i = 1;; ++i) {
                if (__atomic_load_n(&h[0], __ATOMIC_ACQUIRE)) return __atomic_load_n(&h[1], __ATOMIC_RELAXED);
                __builtin_ia32_pause();
                if (i % 64 == 0 && std::chrono::steady_clock::now() > until) break;
            }
            if (hipStreamSynchronize(stream) != hipSuccess)
                throw std::runtime_error(std::string("hipStreamSynchronize: ") +
                                         hipGetErrorString(hipGetLastError()));
            if (__atomic_load_n(&h[0], __ATOMIC_ACQUIRE)) return __atomic_load_n(&h[1], __ATOMIC_RELAXED);
        }
    }
    return work.select(0, 0).item<int64_t>();
}

// Waits for the call and raises ValueError for status bits, as walks.py's
// check=True does.
void check_status(const at::Tensor& work, hipStream_t stream, const char* what) {
    const int64_t bits = read_status(work, stream);
    if (bits == 0) return;
    std::string msg = std::string(what) + ": ";
    if (bits & MLXC_STATUS_BAD_NODE) msg += "a start or col entry is outside [0, num_nodes)";
    if (bits & MLXC_STATUS_BAD_ROW) {
        if (bits & MLXC_STATUS_BAD_NODE) msg += "; ";
        msg += "rowptr is malformed (an entry outside [0, num_edges] or decreasing)";
    }
    throw py::value_error(msg);
}

py::object outputs(const at::Tensor& n_out, const at::Tensor& e_out, bool return_edges) {
    if (return_edges) return py::make_tuple(n_out, e_out);
    return py::cast(n_out);
}

// random_walk(rowptr, col, start, rand or None, walk_length, seed or None,
// check, return_edges, int32_out) -> walks, (walks, edges) or None.
py::object random_walk(const at::Tensor& rowptr, const at::Tensor& col, const at::Tensor& start,
                       std::optional<at::Tensor> rand, int64_t walk_length,
                       std::optional<uint64_t> seed, bool check, bool return_edges,
                       bool int32_out) {
    if (!rowptr.is_cuda() || rowptr.dim() != 1 || rowptr.numel() < 1 || col.dim() != 1 ||
        start.dim() != 1 || walk_length < 0 || walk_length > INT32_MAX - 1 ||
        rand.has_value() == seed.has_value())
        return py::none();
    const at::Device device = rowptr.device();
    if (device.index() != c10::hip::current_device()) return py::none();
    if (!usable(rowptr, at::kLong, device) || !usable(col, at::kLong, device) ||
        !usable(start, at::kLong, device))
        return py::none();
    const int64_t N = start.numel(), L = walk_length;
    if (rand && (!usable(*rand, at::kFloat, device) || rand->numel() != N * L)) return py::none();
    const int64_t V = rowptr.numel() - 1, E = col.numel();
    const auto dtype = int32_out ? at::kInt : at::kLong;
    const auto opts = at::TensorOptions().dtype(dtype).device(device);
    at::Tensor n_out = at::empty({N, L + 1}, opts);
    at::Tensor e_out = return_edges ? at::empty({N, L}, opts) : at::Tensor();
    const size_t ws = mlxc_random_walk_workspace_bytes(V, E, N, static_cast<int32_t>(L));
    at::Tensor work = at::empty({static_cast<int64_t>((ws + 7) / 8)},
                                at::TensorOptions().dtype(at::kLong).device(device));
    hipStream_t stream = at::hip::getCurrentHIPStream().stream();
    const int out_type = int32_out ? MLXC_OUT_INT32 : MLXC_OUT_INT64;
    int rc;
    if (rand)
        rc = mlxc_random_walk(
            static_cast<const int64_t*>(data_or_null(rowptr)), V,
            static_cast<const int64_t*>(data_or_null(col)), E,
            static_cast<const int64_t*>(data_or_null(start)), N,
            static_cast<const float*>(data_or_null(*rand)), static_cast<int32_t>(L),
            n_out.numel() ? n_out.data_ptr() : nullptr,
            return_edges && e_out.numel() ? e_out.data_ptr() : nullptr, out_type,
            work.data_ptr(), static_cast<size_t>(work.numel()) * 8, stream);
    else
        rc = mlxc_random_walk_seeded(
            static_cast<const int64_t*>(data_or_null(rowptr)), V,
            static_cast<const int64_t*>(data_or_null(col)), E,
            static_cast<const int64_t*>(data_or_null(start)), N, static_cast<int32_t>(L), *seed,
            0, n_out.numel() ? n_out.data_ptr() : nullptr,
            return_edges && e_out.numel() ? e_out.data_ptr() : nullptr, out_type,
            work.data_ptr(), static_cast<size_t>(work.numel()) * 8, stream);
    if (rc != MLXC_OK) raise_code(rc, "random_walk");
    if (check) check_status(work, stream, "random_walk");
    return outputs(n_out, e_out, return_edges);
}

// rejection_sampling(rowptr, col, start, walk_length, p, q, seed, rule, rows,
// check, return_edges, int32_out) -> walks, (walks, edges) or None.
py::object rejection_sampling(const at::Tensor& rowptr, const at::Tensor& col,
                              const at::Tensor& start, int64_t walk_length, double p, double q,
                              uint64_t seed, int32_t rule, int32_t rows, bool check,
                              bool return_edges, bool int32_out) {
    if (!rowptr.is_cuda() || rowptr.dim() != 1 || rowptr.numel() < 1 || col.dim() != 1 ||
        start.dim() != 1 || walk_length < 0 || walk_length > INT32_MAX - 1)
        return py::none();
    const at::Device device = rowptr.device();
    if (device.index() != c10::hip::current_device()) return py::none();
    if (!usable(rowptr, at::kLong, device) || !usable(col, at::kLong, device) ||
        !usable(start, at::kLong, device))
        return py::none();
    const int64_t N = start.numel(), L = walk_length;
    const int64_t V = rowptr.numel() - 1, E = col.numel();
    const auto dtype = int32_out ? at::kInt : at::kLong;
    const auto opts = at::TensorOptions().dtype(dtype).device(device);
    at::Tensor n_out = at::empty({N, L + 1}, opts);
    at::Tensor e_out = return_edges ? at::empty({N, L}, opts) : at::Tensor();
    const size_t ws = mlxc_rejection_sampling_workspace_bytes(V, E, N, static_cast<int32_t>(L), p,
                                                              q, rule);
    at::Tensor work = at::empty({static_cast<int64_t>((ws + 7) / 8)},
                                at::TensorOptions().dtype(at::kLong).device(device));
    hipStream_t stream = at::hip::getCurrentHIPStream().stream();
    const int rc = mlxc_rejection_sampling(
        static_cast<const int64_t*>(data_or_null(rowptr)), V,
        static_cast<const int64_t*>(data_or_null(col)), E,
        static_cast<const int64_t*>(data_or_null(start)), N, static_cast<int32_t>(L), p, q, seed,
        0, rule, rows, n_out.numel() ? n_out.data_ptr() : nullptr,
        return_edges && e_out.numel() ? e_out.data_ptr() : nullptr,
        int32_out ? MLXC_OUT_INT32 : MLXC_OUT_INT64, work.data_ptr(),
        static_cast<size_t>(work.numel()) * 8, stream);
    if (rc != MLXC_OK) raise_code(rc, "rejection_sampling");
    if (check) check_status(work, stream, "rejection_sampling");
    return outputs(n_out, e_out, return_edges);
}

}  // namespace

PYBIND11_MODULE(_mlxc_torch, m) {
    m.doc() = "Compiled fast path of mlx_cluster_amd.random_walk / rejection_sampling";
    m.def("random_walk", &random_walk);
    m.def("rejection_sampling", &rejection_sampling);
}
