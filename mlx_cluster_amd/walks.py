"""Python surface of the random-walk path, mirroring mlx_cluster's.

Reference interface (vinayhpandya/mlx_cluster):
  random_walk(rowptr, col, start, rand, walk_length, *, stream=None)
      /root/reference/bindings.cpp:12-33, op at
      /root/reference/random_walks/RandomWalk.cpp:138-148
  rejection_sampling(rowptr, col, start, walk_length, p, q, *, stream=None)
      /root/reference/bindings.cpp:35-63, op at
      /root/reference/random_walks/BiasedRandomWalk.cpp:183-193

Same names, positional order and keyword-only `stream`.  Arrays are torch
tensors on a ROCm device (numpy arrays and CPU tensors are copied to the
current device).  Both functions return the node sequences, an int64 tensor
[num_walks, walk_length + 1], as the reference ops do (they discard the edge
output, RandomWalk.cpp:147); `return_edges=True` also returns the edge ids,
and `out_dtype=torch.int32` gives both as int32, with half the bytes.

Every walk runs in the library libmlxc.so: on the GPU through its HIP
kernels, or, for stream='cpu' (the reference's eval_cpu), through its host
twins on CPU threads, which give bit-identical results.  There is no
fallback from one to the other.
"""
from __future__ import annotations

import contextlib
import numbers
import os
from typing import Optional, Tuple, Union

import numpy as np
import torch

from . import _lib

TensorLike = Union[torch.Tensor, np.ndarray]

_RULES = {"ref_chain": _lib.MLXC_RULE_REF_CHAIN, "node2vec": _lib.MLXC_RULE_NODE2VEC_EXACT}

# The compiled fast path (csrc/torch_binding.cpp): the same calls into
# libmlxc.so for the common case (tensors of the right dtype on the current
# device, torch's current stream), without this layer's per-call cost; it
# returns None for any other call.  Without it every call takes the path below.
# It is linked to the in-tree libmlxc.so, so another build selected by
# MLXC_LIB takes the path below for every call.
_fast = None
if os.path.realpath(_lib.LIB_PATH) == os.path.realpath(_lib.IN_TREE_LIB):
    try:
        from . import _mlxc_torch as _fast
    except ImportError:
        _fast = None


# ---------------------------------------------------------------- helpers

def _resolve_device(stream, tensors) -> torch.device:
    if _on_cpu(stream):
        raise ValueError("this operation runs on the GPU only; stream='cpu' is for "
                         "random_walk and rejection_sampling")
    if isinstance(stream, torch.cuda.Stream):
        return stream.device
    if isinstance(stream, (str, torch.device)):  # a GPU named as the stream: run there
        named = torch.device(stream)
        if named.type != "cuda":
            raise ValueError(f"stream names device {named}; expected a GPU or 'cpu'")
        if named.index is not None:
            return named
        if not torch.cuda.is_available():
            raise RuntimeError("mlx_cluster_amd needs a ROCm GPU; none is visible")
        return torch.device("cuda", torch.cuda.current_device())
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("mlx_cluster_amd needs a ROCm GPU; none is visible")
    return torch.device("cuda", torch.cuda.current_device())


# torch's current stream of a device as a raw handle, without building a
# torch.cuda.Stream object (a small call's overhead is mostly the Python layer)
_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _stream_handle(stream, device: torch.device) -> int:
    """hipStream_t for `stream`: None -> torch's current stream on device."""
    _check_stream_arg(stream)
    if _on_cpu(stream) or device.type != "cuda":
        raise ValueError("this operation runs on the GPU only; stream='cpu' is for "
                         "random_walk and rejection_sampling")
    if stream is None:
        if _current_raw_stream is not None:
            return _current_raw_stream(_device_index(device))
        return torch.cuda.current_stream(device).cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return torch.cuda.current_stream(torch.device(stream)).cuda_stream


def _side_stream(stream, device: torch.device) -> Optional[torch.cuda.Stream]:
    """`stream` when a call runs on a torch.cuda.Stream that is not torch's
    current stream of `device`, else None."""
    if isinstance(stream, torch.cuda.Stream) and \
            stream.cuda_stream != torch.cuda.current_stream(device).cuda_stream:
        return stream
    return None


def _enter_side_stream(side: Optional[torch.cuda.Stream], device: torch.device) -> None:
    """A call copies its inputs and allocates its outputs and workspace on
    torch's current stream: the side stream it launches on waits for that
    work first, so no kernel reads a copy still in flight or writes memory
    the allocator handed over while an earlier kernel on the current stream
    still used it."""
    if side is not None:
        side.wait_stream(torch.cuda.current_stream(device))


def _leave_side_stream(side: Optional[torch.cuda.Stream], *tensors) -> None:
    """Marks every device tensor a side-stream call touched as used on that
    stream, so the caching allocator reuses none of them (the workspace and
    input copies are freed when the call returns) before the stream's
    kernels have finished."""
    if side is not None:
        for t in tensors:
            if isinstance(t, torch.Tensor) and t.is_cuda and t.numel():
                t.record_stream(side)


def _on_device(device: torch.device):
    """The library's calls query and launch on the current device: make it
    `device` (a no-op context when it already is)."""
    index = _device_index(device)
    if index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(index)


def _as_tensor(x: TensorLike, dtype: torch.dtype, name: str) -> torch.Tensor:
    """Type checks (no device work): numpy arrays are wrapped, dtypes must match."""
    if isinstance(x, np.ndarray):
        x = torch.from_numpy(x)
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor or numpy.ndarray, got {type(x)!r}")
    if x.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}, got {x.dtype}")
    return x


def _on(x: torch.Tensor, device: torch.device) -> torch.Tensor:
    if x.device != device:
        x = x.to(device)
    return x.contiguous()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _graph(rowptr, col, start):
    rowptr = _as_tensor(rowptr, torch.int64, "rowptr")
    col = _as_tensor(col, torch.int64, "col")
    start = _as_tensor(start, torch.int64, "start")
    if rowptr.dim() != 1 or rowptr.numel() < 1:
        raise ValueError("rowptr must be 1-D with num_nodes + 1 >= 1 entries")
    if col.dim() != 1:
        raise ValueError("col must be 1-D")
    return rowptr, col, start.reshape(-1)


def _check_stream_arg(stream) -> None:
    if stream is not None and not isinstance(stream, (str, torch.device, torch.cuda.Stream)):
        raise TypeError(f"stream must be None, a torch.cuda.Stream or a device, got {type(stream)!r}")
    if isinstance(stream, (str, torch.device)):
        torch.device(stream)  # raises on an unknown device string


def _on_cpu(stream) -> bool:
    """stream='cpu' (or torch.device('cpu')) selects the host evaluation."""
    return isinstance(stream, (str, torch.device)) and torch.device(stream).type == "cpu"


def _threads(threads) -> int:
    if threads is None:
        return 0  # one per hardware thread
    if isinstance(threads, bool) or not isinstance(threads, numbers.Integral) or threads < 1:
        raise ValueError("threads must be None or an int >= 1")
    return min(int(threads), 2**31 - 1)


def _host(x: torch.Tensor) -> torch.Tensor:
    return x.cpu().contiguous()


_OUT_TYPES = {torch.int64: _lib.MLXC_OUT_INT64, torch.int32: _lib.MLXC_OUT_INT32}


def _out_type(out_dtype) -> int:
    if out_dtype not in _OUT_TYPES:
        raise TypeError(f"out_dtype must be torch.int64 or torch.int32, got {out_dtype!r}")
    return _OUT_TYPES[out_dtype]


def _walk_length(walk_length) -> int:
    if isinstance(walk_length, bool) or not isinstance(walk_length, numbers.Integral):
        raise TypeError("walk_length must be an int")
    walk_length = int(walk_length)
    if walk_length < 0:
        raise ValueError("walk_length must be >= 0")
    if walk_length > 2**31 - 2:
        raise ValueError("walk_length too large")
    return walk_length


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Device workspace of at least nbytes (int64 words, so 16-byte aligned
    from torch's allocator); torch's caching allocator recycles it."""
    return torch.empty((int(nbytes) + 7) // 8, dtype=torch.int64, device=device)


def _raise_status(work: torch.Tensor, stream, what: str) -> None:
    if isinstance(stream, torch.cuda.Stream):
        stream.synchronize()  # the kernel ran there, not on torch's current stream
    _raise_bits(int(work[0].item()), what)


def _raise_bits(bits: int, what: str) -> None:
    if bits == 0:
        return
    reasons = []
    if bits & _lib.MLXC_STATUS_BAD_NODE:
        reasons.append("a start or col entry is outside [0, num_nodes)")
    if bits & _lib.MLXC_STATUS_BAD_ROW:
        reasons.append("rowptr is malformed (an entry outside [0, num_edges] or decreasing)")
    raise ValueError(f"{what}: " + "; ".join(reasons))


def _walk_offset(walk_offset) -> int:
    if isinstance(walk_offset, bool) or not isinstance(walk_offset, numbers.Integral):
        raise TypeError("walk_offset must be an int")
    if walk_offset < 0 or walk_offset >= 2**63:
        raise ValueError("walk_offset must lie in [0, 2^63)")
    return int(walk_offset)


def _memory_budget(budget) -> Optional[int]:
    if budget is None:
        return None
    if isinstance(budget, bool) or not isinstance(budget, numbers.Integral) or budget < 1:
        raise ValueError("memory_budget must be None or a positive int (bytes)")
    return int(budget)


def _available_bytes(device: torch.device) -> int:
    """Device memory a call can take: the driver's free memory plus what
    torch's caching allocator holds unused."""
    index = _device_index(device)
    free, _ = torch.cuda.mem_get_info(index)
    return int(free) + torch.cuda.memory_reserved(index) - torch.cuda.memory_allocated(index)


# Smallest workspace a walk entry point accepts (MLXC_WORK_WORDS int64
# words): the direct kernels, which read the CSR arrays as they are.
_MIN_WORKSPACE = _lib.MLXC_WORK_WORDS * 8
# Chunks of a chunked call are whole multiples of this many walks, so every
# chunk's rows of the rand tensor and of the staging outputs start 16-byte
# aligned (the windowed kernels' requirement).
_CHUNK_ALIGN = 64


def _plan(N: int, row_bytes: int, ws_query, budget: int):
    """How a call of N walks runs within `budget` bytes of device memory for
    its outputs (row_bytes per walk) and workspace (ws_query(n) bytes for n
    walks at the fastest layout; any smaller workspace of at least
    _MIN_WORKSPACE bytes runs too, at a slower layout with the same results).

    Returns ("device", None, ws): one call with device outputs and a
    workspace of ws bytes; or ("host", chunk, ws): chunks of `chunk` walks
    into two device staging buffers, copied into pinned host outputs."""
    out = N * row_bytes
    if out + ws_query(N) <= budget:
        return "device", None, ws_query(N)
    if out + _MIN_WORKSPACE <= budget:
        return "device", None, (budget - out) // 16 * 16
    cost = lambda c: 2 * c * row_bytes + ws_query(c)
    hi = N // _CHUNK_ALIGN
    if hi >= 1 and cost(_CHUNK_ALIGN) <= budget:
        lo = 1  # the largest multiple k of _CHUNK_ALIGN with cost(k * _CHUNK_ALIGN) <= budget
        while lo < hi:
            mid = (lo + hi + 1) // 2
            if cost(mid * _CHUNK_ALIGN) <= budget:
                lo = mid
            else:
                hi = mid - 1
        chunk = lo * _CHUNK_ALIGN
        return "host", chunk, ws_query(chunk)
    chunk = min(N, (budget - _MIN_WORKSPACE) // (2 * row_bytes))
    if chunk >= _CHUNK_ALIGN:
        chunk -= chunk % _CHUNK_ALIGN
    if chunk < 1:
        raise ValueError(f"memory_budget of {budget} bytes holds no chunk: one walk needs "
                         f"{2 * row_bytes + _MIN_WORKSPACE} bytes (two staging rows and the "
                         f"minimal workspace)")
    return "host", chunk, min(ws_query(chunk), (budget - 2 * chunk * row_bytes) // 16 * 16)


def _run_walks(device, stream, handle, N: int, L: int, out_dtype, return_edges: bool,
               ws_query, launch, budget: Optional[int], check: bool, what: str, inputs):
    """Runs a walk call on the device.  launch(i0, n, n_ptr, e_ptr, ws_ptr,
    ws_bytes) enqueues walks [i0, i0 + n) of the call on `handle` and returns
    the library's code.  Without a budget the call runs once, with device
    outputs and the fastest workspace; when that allocation fails, or when
    the outputs and workspace would exceed `budget` bytes, _plan decides."""
    esize = 8 if out_dtype == torch.int64 else 4
    row_bytes = (2 * L + 1 if return_edges else L + 1) * esize
    if budget is None:
        try:
            return _run_once(device, stream, N, L, out_dtype, return_edges, ws_query(N), launch,
                             check, what, inputs)
        except torch.cuda.OutOfMemoryError:
            budget = _available_bytes(device)
    mode, chunk, ws_bytes = _plan(N, row_bytes, ws_query, budget)
    if mode == "device":
        return _run_once(device, stream, N, L, out_dtype, return_edges, ws_bytes, launch, check,
                         what, inputs)
    return _run_chunked(device, stream, N, L, out_dtype, return_edges, chunk, ws_bytes, launch,
                        check, what, inputs)


def _run_once(device, stream, N, L, out_dtype, return_edges, ws_bytes, launch, check, what,
              inputs):
    n_out = torch.empty((N, L + 1), dtype=out_dtype, device=device)
    e_out = torch.empty((N, L), dtype=out_dtype, device=device) if return_edges else None
    work = _workspace(ws_bytes, device)
    side = _side_stream(stream, device)
    _enter_side_stream(side, device)
    with _on_device(device):
        rc = launch(0, N, _ptr(n_out), _ptr(e_out) if return_edges else None, work.data_ptr(),
                    work.numel() * 8)
    _leave_side_stream(side, *inputs, n_out, e_out, work)
    _lib.check(rc, what)
    if check:
        _raise_status(work, stream, what)
    return n_out, e_out


def _run_chunked(device, stream, N, L, out_dtype, return_edges, chunk, ws_bytes, launch, check,
                 what, inputs):
    """Walks in chunks of `chunk`, each written into one of two device staging
    buffers and copied on a copy stream into pinned host outputs while the
    next chunk runs.  Synchronises before returning (the outputs are host
    memory); the status bits of every chunk are OR-ed on the device."""
    n_host = torch.empty((N, L + 1), dtype=out_dtype, pin_memory=True)
    e_host = torch.empty((N, L), dtype=out_dtype, pin_memory=True) if return_edges else None
    compute = stream if isinstance(stream, torch.cuda.Stream) else torch.cuda.current_stream(device)
    _enter_side_stream(_side_stream(stream, device), device)
    with _on_device(device), torch.cuda.stream(compute):
        n_stage = torch.empty((2, chunk, L + 1), dtype=out_dtype, device=device)
        e_stage = (torch.empty((2, chunk, L), dtype=out_dtype, device=device) if return_edges
                   else None)
        work = _workspace(ws_bytes, device)
        status = torch.zeros(1, dtype=torch.int64, device=device)
        copy = torch.cuda.Stream(device)
        copied = [None, None]  # copy-stream events after which a staging buffer is free
        for k, i0 in enumerate(range(0, N, chunk)):
            n, b = min(chunk, N - i0), k % 2
            if copied[b] is not None:
                compute.wait_event(copied[b])
            rc = launch(i0, n, n_stage[b].data_ptr(),
                        e_stage[b].data_ptr() if return_edges else None, work.data_ptr(),
                        work.numel() * 8)
            if rc != _lib.MLXC_OK:
                copy.synchronize()
                _lib.check(rc, what)
            status.bitwise_or_(work[:1])
            done = torch.cuda.Event()
            done.record(compute)
            copy.wait_event(done)
            with torch.cuda.stream(copy):
                n_host[i0:i0 + n].copy_(n_stage[b, :n], non_blocking=True)
                if return_edges:
                    e_host[i0:i0 + n].copy_(e_stage[b, :n], non_blocking=True)
                copied[b] = torch.cuda.Event()
                copied[b].record(copy)
        copy.synchronize()
    if check:
        _raise_bits(int(status.item()), what)
    return n_host, e_host


# ------------------------------------------------------------------- API

def random_walk(rowptr: TensorLike, col: TensorLike, start: TensorLike,
                rand: Optional[TensorLike], walk_length: int, *, stream=None,
                return_edges: bool = False, check: bool = True, seed: Optional[int] = None,
                threads: Optional[int] = None, out_dtype: torch.dtype = torch.int64,
                walk_offset: int = 0, memory_budget: Optional[int] = None
                ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Uniform random walks over a CSR graph.

    Mirrors mlx_cluster.random_walk (/root/reference/bindings.cpp:12-33;
    semantics /root/reference/random_walks/RandomWalk.cpp:41-60).

    Args:
        rowptr: int64 [num_nodes + 1] CSR row pointer.
        col: int64 [num_edges] CSR column indices.
        start: int64 [num_walks] start nodes (any shape; flattened).
        rand: float32 with num_walks * walk_length uniforms in [0, 1); walk n
            reads rand.view(-1)[n * walk_length + l] at step l.  None with
            `seed` set: the kernels generate the uniforms themselves,
            bit-identical to rand = philox_uniform((num_walks, walk_length),
            seed), without the rand tensor's memory traffic.
        walk_length: steps per walk (>= 0).
        stream: None (torch's current stream), a torch.cuda.Stream or a
            device.  On a torch.cuda.Stream the kernels run after the work
            already queued on torch's current stream (where inputs are
            copied and outputs allocated), and every tensor of the call is
            recorded as used there.  'cpu' evaluates on CPU threads (the
            reference's eval_cpu) with results bit-identical to the GPU's;
            inputs are copied to host memory and outputs are CPU tensors.
        return_edges: also return the edge ids [num_walks, walk_length]
            (-1 where the walk stayed in a node of out-degree 0), the
            reference's discarded second output (RandomWalk.cpp:58).
        check: synchronise and raise ValueError if a start/col index or a
            rowptr entry was out of range (the reference reads out of bounds
            there).  With check=False the call stays asynchronous.
        seed: key of the generated uniforms when rand is None.
        threads: the most CPU threads stream='cpu' may use (None: one per
            hardware thread; small calls use fewer); ignored on the GPU.
        out_dtype: torch.int64 (the reference's output) or torch.int32, a
            compact output with half the bytes (node ids, and edge ids with
            return_edges, must be below 2^31).
        walk_offset: with seed, the index of this call's first walk in a
            larger batch: walk n draws the uniforms of walk walk_offset + n,
            so the call on start[i0:i1] with walk_offset=i0 returns rows
            i0 .. i1-1 of the whole batch's call, bit for bit.  (With a rand
            tensor, pass the slice's rows of rand instead.)
        memory_budget: bytes of device memory the call may allocate for its
            outputs and workspace (None: whatever it needs, and if that
            allocation fails, what the device has free).  Outputs that fit
            stay on the device, with the workspace shrunk to the rest if
            needed (a slower kernel layout, the same walks).  Outputs that do
            not fit are computed in chunks of walks, each with its walk
            offset, through two device staging buffers, and returned in
            pinned host memory (the call then synchronises).  Ignored for
            stream='cpu'.

    Returns:
        [num_walks, walk_length + 1] node sequences (and edge ids) of out_dtype.
    """
    if (_fast is not None and stream is None and walk_offset == 0 and memory_budget is None and
            type(rowptr) is torch.Tensor and type(col) is torch.Tensor and
            type(start) is torch.Tensor and type(walk_length) is int and
            (rand is None or type(rand) is torch.Tensor) and
            (seed is None or type(seed) is int) and
            (out_dtype is torch.int64 or out_dtype is torch.int32)):
        res = _fast.random_walk(rowptr, col, start, rand, walk_length,
                                None if seed is None else seed & (2**64 - 1), bool(check),
                                bool(return_edges), out_dtype is torch.int32)
        if res is not None:
            return res
    L = _walk_length(walk_length)
    otype = _out_type(out_dtype)
    offset = _walk_offset(walk_offset)
    budget = _memory_budget(memory_budget)
    _check_stream_arg(stream)
    rowptr, col, start = _graph(rowptr, col, start)
    N = start.numel()
    if rand is None:
        if seed is None:
            raise ValueError("rand is None: pass seed= to have the kernels generate the uniforms")
        seed = int(seed) & (2**64 - 1)
    else:
        if seed is not None:
            raise ValueError("pass either rand or seed, not both")
        if offset:
            raise ValueError("walk_offset applies to generated uniforms (seed=); with a rand "
                             "tensor, pass the rows of rand that belong to these walks")
        rand = _as_tensor(rand, torch.float32, "rand")
        if rand.numel() != N * L:
            raise ValueError(f"rand must hold num_walks * walk_length = {N * L} values, "
                             f"got {rand.numel()}")
    if _on_cpu(stream):
        rowptr, col, start = (_host(t) for t in (rowptr, col, start))
        n_out = torch.empty((N, L + 1), dtype=out_dtype)
        e_out = torch.empty((N, L), dtype=out_dtype) if return_edges else None
        status = _lib.ctypes.c_int64(0)
        graph = (_ptr(rowptr), rowptr.numel() - 1, _ptr(col), col.numel(), _ptr(start), N)
        outs = (_ptr(n_out), _ptr(e_out), otype, _threads(threads),
                _lib.ctypes.addressof(status))
        if rand is None:
            rc = _lib.load().mlxc_random_walk_seeded_cpu(*graph, L, seed, offset, *outs)
        else:
            rand = _host(rand)
            rc = _lib.load().mlxc_random_walk_cpu(*graph, _ptr(rand), L, *outs)
        _lib.check(rc, "random_walk")
        if check:
            _raise_bits(int(status.value), "random_walk")
        return (n_out, e_out) if return_edges else n_out
    device = _resolve_device(stream, (rowptr, col, start, rand))
    handle = _stream_handle(stream, device)
    rowptr, col, start = (_on(t, device) for t in (rowptr, col, start))
    if rand is not None:
        rand = _on(rand, device)
    lib = _lib.load()
    V, E = rowptr.numel() - 1, col.numel()
    rowptr_p, col_p = _ptr(rowptr), _ptr(col)
    start_p = start.data_ptr() if N else None
    rand_p = rand.data_ptr() if rand is not None and rand.numel() else None

    def launch(i0, n, n_p, e_p, ws_p, ws_bytes):
        s_p = start_p + 8 * i0 if start_p else None
        if rand is None:
            return lib.mlxc_random_walk_seeded(rowptr_p, V, col_p, E, s_p, n, L, seed,
                                               offset + i0, n_p, e_p, otype, ws_p, ws_bytes,
                                               handle)
        r_p = rand_p + 4 * L * i0 if rand_p else None
        return lib.mlxc_random_walk(rowptr_p, V, col_p, E, s_p, n, r_p, L, n_p, e_p, otype, ws_p,
                                    ws_bytes, handle)

    n_out, e_out = _run_walks(
        device, stream, handle, N, L, out_dtype, return_edges,
        lambda n: lib.mlxc_random_walk_workspace_bytes(V, E, n, L), launch, budget, check,
        "random_walk", (rowptr, col, start, rand))
    return (n_out, e_out) if return_edges else n_out


def csr_check(rowptr: TensorLike, col: TensorLike, *, stream=None) -> int:
    """MLXC_CSR_* bits of a CSR graph, computed on the device (synchronous):
    1 malformed rowptr, 2 a col entry outside [0, num_nodes), 4 some row not
    sorted, 8 (checked on well-formed graphs with sorted rows) some entry
    (u, v) without its reverse (v, u), i.e. symmetric=True would not hold."""
    _check_stream_arg(stream)
    rowptr, col, _ = _graph(rowptr, col, torch.empty(0, dtype=torch.int64))
    device = _resolve_device(stream, (rowptr, col))
    handle = _stream_handle(stream, device)
    rowptr, col = _on(rowptr, device), _on(col, device)
    work = _workspace(_lib.MLXC_WORK_WORDS * 8, device)
    flags = _lib.ctypes.c_int32(0)
    side = _side_stream(stream, device)
    _enter_side_stream(side, device)
    with _on_device(device):
        rc = _lib.load().mlxc_csr_check(_ptr(rowptr), rowptr.numel() - 1, _ptr(col), col.numel(),
                                        work.data_ptr(), work.numel() * 8,
                                        _lib.ctypes.addressof(flags), handle)
    _leave_side_stream(side, rowptr, col, work)
    _lib.check(rc, "csr_check")
    return int(flags.value)


def rejection_sampling(rowptr: TensorLike, col: TensorLike, start: TensorLike,
                       walk_length: int, p: float, q: float, *, stream=None,
                       seed: Optional[int] = None, rule: str = "ref_chain",
                       rows_sorted: Optional[bool] = None, return_edges: bool = False,
                       check: bool = True, threads: Optional[int] = None,
                       out_dtype: torch.dtype = torch.int64, symmetric: bool = False,
                       walk_offset: int = 0, memory_budget: Optional[int] = None
                       ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """node2vec random walks by rejection sampling.

    Mirrors mlx_cluster.rejection_sampling (/root/reference/bindings.cpp:35-63;
    semantics /root/reference/random_walks/BiasedRandomWalk.cpp:52-100),
    which has no GPU implementation in the reference (:150-155).

    Args:
        rowptr, col, start, walk_length: as in random_walk.
        p: return parameter (likelihood of revisiting the previous node).
        q: in-out parameter (breadth- versus depth-first).
        stream: as in random_walk.
        seed: key of the Philox4x32-10 stream the walk draws from (the
            reference uses libc rand()).  None draws one from torch's default
            CPU generator, so torch.manual_seed makes runs repeatable.
        rule: 'ref_chain' reproduces the reference's acceptance chain
            (BiasedRandomWalk.cpp:86-91) term for term; 'node2vec' is the
            analytic node2vec rule (accept with probability 1/p, 1 or 1/q,
            normalised).  They agree whenever q >= max(p, 1).
        rows_sorted: whether every CSR row is sorted ascending (sorted rows
            are searched, unsorted ones scanned as the reference does).  None
            lets the call check the rows on the device as part of its
            preparation pass, which also validates the whole graph (a
            malformed graph raises ValueError when check=True).
        return_edges, check, threads, out_dtype: as in random_walk.
        symmetric: the caller promises the graph is symmetric (every (u, v)
            has its (v, u), as to_csr(symmetrize=True) makes): the neighbour
            test then searches the shorter of row(x) and row(t), which gives
            the same answer there.  False (the default) searches row(x), as
            the reference does; on a graph that is not symmetric True gives
            unspecified walks.  csr_check(rowptr, col) & MLXC_CSR_ASYMMETRIC
            (8) tells whether the promise holds (for sorted rows).
        walk_offset: the index of this call's first walk in a larger batch:
            walk n draws from the Philox stream of walk walk_offset + n, so
            the call on start[i0:i1] with walk_offset=i0 (and the same seed)
            returns rows i0 .. i1-1 of the whole batch's call, bit for bit.
        memory_budget: as in random_walk.  A workspace shrunk to fit runs
            the edge records without hub bitmaps, then the CSR mode, then the
            direct kernel: the same walks each way.
    """
    L = _walk_length(walk_length)
    otype = _out_type(out_dtype)
    offset = _walk_offset(walk_offset)
    budget = _memory_budget(memory_budget)
    p, q = float(p), float(q)
    if not (np.isfinite(p) and np.isfinite(q) and p > 0 and q > 0):
        raise ValueError("p and q must be finite and > 0")
    if rule not in _RULES:
        raise ValueError(f"rule must be one of {sorted(_RULES)}")
    _check_stream_arg(stream)
    rowptr, col, start = _graph(rowptr, col, start)
    if seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    seed = int(seed) & (2**64 - 1)
    rows = (_lib.MLXC_ROWS_DETECT if rows_sorted is None else
            _lib.MLXC_ROWS_SORTED if rows_sorted else _lib.MLXC_ROWS_UNSORTED)
    if symmetric:
        rows |= _lib.MLXC_ROWS_SYMMETRIC
    if (_fast is not None and stream is None and walk_offset == 0 and memory_budget is None and
            type(rowptr) is torch.Tensor and type(col) is torch.Tensor and
            type(start) is torch.Tensor and (out_dtype is torch.int64 or out_dtype is torch.int32)):
        res = _fast.rejection_sampling(rowptr, col, start, L, p, q, seed, _RULES[rule], rows,
                                       bool(check), bool(return_edges), out_dtype is torch.int32)
        if res is not None:
            return res
    N = start.numel()
    if _on_cpu(stream):
        rowptr, col, start = (_host(t) for t in (rowptr, col, start))
        n_out = torch.empty((N, L + 1), dtype=out_dtype)
        e_out = torch.empty((N, L), dtype=out_dtype) if return_edges else None
        status = _lib.ctypes.c_int64(0)
        rc = _lib.load().mlxc_rejection_sampling_cpu(
            _ptr(rowptr), rowptr.numel() - 1, _ptr(col), col.numel(), _ptr(start), N, L,
            p, q, seed, offset, _RULES[rule], rows, _ptr(n_out), _ptr(e_out), otype,
            _threads(threads), _lib.ctypes.addressof(status))
        _lib.check(rc, "rejection_sampling")
        if check:
            _raise_bits(int(status.value), "rejection_sampling")
        return (n_out, e_out) if return_edges else n_out
    device = _resolve_device(stream, (rowptr, col, start))
    handle = _stream_handle(stream, device)
    rowptr, col, start = (_on(t, device) for t in (rowptr, col, start))
    lib = _lib.load()
    V, E, rid = rowptr.numel() - 1, col.numel(), _RULES[rule]
    rowptr_p, col_p = _ptr(rowptr), _ptr(col)
    start_p = start.data_ptr() if N else None

    def launch(i0, n, n_p, e_p, ws_p, ws_bytes):
        s_p = start_p + 8 * i0 if start_p else None
        return lib.mlxc_rejection_sampling(rowptr_p, V, col_p, E, s_p, n, L, p, q, seed,
                                           offset + i0, rid, rows, n_p, e_p, otype, ws_p,
                                           ws_bytes, handle)

    n_out, e_out = _run_walks(
        device, stream, handle, N, L, out_dtype, return_edges,
        lambda n: lib.mlxc_rejection_sampling_workspace_bytes(V, E, n, L, p, q, rid), launch,
        budget, check, "rejection_sampling", (rowptr, col, start))
    return (n_out, e_out) if return_edges else n_out


def philox_uniform(shape, seed: int, *, device=None, stream=None) -> torch.Tensor:
    """float32 tensor of Philox4x32-10 uniforms in [0, 1 - 2^-24].

    Element i (row-major) is (w >> 8) * 2^-24 with w word i % 4 of
    Philox(key = seed, counter = (i // 4, 0)).  A seeded stand-in for the
    mx.random.uniform call that makes the reference tests' rand tensor
    (/root/reference/tests/test_random_walk.py:31).
    """
    if isinstance(shape, numbers.Integral):
        shape = (int(shape),)
    _check_stream_arg(stream)
    dev = torch.device(device) if device is not None else _resolve_device(stream, ())
    handle = _stream_handle(stream, dev)
    out = torch.empty(tuple(shape), dtype=torch.float32, device=dev)
    side = _side_stream(stream, dev)
    _enter_side_stream(side, dev)
    with _on_device(dev):
        rc = _lib.load().mlxc_philox_uniform(_ptr(out), out.numel(), int(seed) & (2**64 - 1), handle)
    _leave_side_stream(side, out)
    _lib.check(rc, "philox_uniform")
    return out
