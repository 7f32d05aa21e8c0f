"""CSR construction from an edge list, in libmlxc.so.

The reference's tests build their CSR on the host: sort the edge index, then
rowptr from np.unique(row, return_counts=True) plus a cumulative sum
(/root/reference/tests/test_random_walk.py:23-28).  np.unique skips nodes with
no out-edges, so that rowptr is only valid when every node has one; here
rowptr has an entry for every node, so nodes of out-degree 0 keep their
(empty) rows — the absorbing nodes the walks expect.

Edge lists on a GPU are sorted there by mlxc_csr_build (a radix sort in HIP,
csrc/csr_build.hip); CPU edge lists by its host twin mlxc_csr_build_cpu.
"""
from __future__ import annotations

import ctypes
import numbers
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib
from .walks import (_check_stream_arg, _enter_side_stream, _leave_side_stream, _on_device,
                    _side_stream, _stream_handle, _workspace)


def to_csr(edge_index, num_nodes: Optional[int] = None, *, symmetrize: bool = False,
           dedup: bool = False, device=None, stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(rowptr, col) int64 of a directed edge list, rows sorted by (row, col).

    Args:
        edge_index: int [2, E] (row, col) pairs; torch tensor or numpy array.
        num_nodes: node count V (default: max id + 1); at most 2^32.
        symmetrize: add every reversed edge (undirected graphs).
        dedup: merge duplicate edges (the reference's pipeline keeps them).
        device: where to build (default: edge_index's device).  A GPU builds
            with mlxc_csr_build, the CPU with mlxc_csr_build_cpu.
        stream: GPU only: a torch.cuda.Stream to run on (default: torch's
            current stream); without device=, the build runs on the
            stream's device.  The call synchronises with it once, to read
            the entry count and the id check.

    Raises ValueError when an id lies outside [0, num_nodes).
    """
    if isinstance(edge_index, np.ndarray):
        edge_index = torch.from_numpy(edge_index)
    if not isinstance(edge_index, torch.Tensor) or edge_index.dim() != 2 or edge_index.shape[0] != 2:
        raise ValueError("edge_index must be a [2, E] tensor or array")
    if edge_index.dtype.is_floating_point or edge_index.dtype.is_complex or \
            edge_index.dtype == torch.bool:
        raise TypeError(f"edge_index must hold integers, got {edge_index.dtype}")
    _check_stream_arg(stream)
    if stream is not None and not isinstance(stream, torch.cuda.Stream):
        raise TypeError("to_csr: stream must be None or a torch.cuda.Stream (name the build's "
                        "device with device=)")
    if device is None and stream is not None:
        device = stream.device  # build where the stream runs
    if device is not None:
        edge_index = edge_index.to(device)
    if stream is not None and edge_index.device != stream.device:
        raise ValueError(f"to_csr: stream runs on {stream.device}, the build on "
                         f"{edge_index.device}")
    row = edge_index[0].to(torch.int64).contiguous()
    col = edge_index[1].to(torch.int64).contiguous()
    E = row.numel()
    if num_nodes is None:
        num_nodes = int(torch.maximum(row.max(), col.max()).item()) + 1 if E else 0
    if isinstance(num_nodes, bool) or not isinstance(num_nodes, numbers.Integral):
        raise TypeError("num_nodes must be an int")
    V = int(num_nodes)
    if V < 0:
        raise ValueError("num_nodes must be >= 0")
    flags = ((_lib.MLXC_CSR_SYMMETRIZE if symmetrize else 0) |
             (_lib.MLXC_CSR_DEDUP if dedup else 0))
    total = 2 * E if symmetrize else E
    dev = row.device
    lib = _lib.load()
    rowptr = torch.empty(V + 1, dtype=torch.int64, device=dev)
    col_out = torch.empty(total, dtype=torch.int64, device=dev)
    if dev.type == "cpu":
        count, status = ctypes.c_int64(0), ctypes.c_int64(0)
        rc = lib.mlxc_csr_build_cpu(row.data_ptr() if E else None, col.data_ptr() if E else None,
                                    E, V, flags, rowptr.data_ptr(),
                                    col_out.data_ptr() if total else None,
                                    ctypes.addressof(count), ctypes.addressof(status))
        _lib.check(rc, "to_csr")
        bits, n = int(status.value), int(count.value)
    else:
        handle = _stream_handle(stream, dev)
        nbytes = lib.mlxc_csr_build_workspace_bytes(V, E, flags)
        if nbytes == 0:
            raise ValueError("to_csr: num_nodes or the edge count is out of range")
        work = _workspace(nbytes, dev)
        side = _side_stream(stream, dev)
        _enter_side_stream(side, dev)
        with _on_device(dev):
            rc = lib.mlxc_csr_build(row.data_ptr() if E else None, col.data_ptr() if E else None,
                                    E, V, flags, rowptr.data_ptr(),
                                    col_out.data_ptr() if total else None, work.data_ptr(),
                                    work.numel() * 8, handle)
        _leave_side_stream(side, row, col, rowptr, col_out, work)
        _lib.check(rc, "to_csr")
        if isinstance(stream, torch.cuda.Stream):
            stream.synchronize()
        bits, n = (int(x) for x in work[:2].tolist())
        del work
    if bits & _lib.MLXC_STATUS_BAD_NODE:
        raise ValueError("edge_index holds ids outside [0, num_nodes)")
    return rowptr, col_out[:n]
