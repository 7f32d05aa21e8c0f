"""CSR construction from an edge list, on the device.

The reference's tests build their CSR on the host: sort the edge index, then
rowptr from np.unique(row, return_counts=True) plus a cumulative sum
(/root/reference/tests/test_random_walk.py:23-28).  np.unique skips nodes with
no out-edges, so that rowptr is only valid when every node has one; here the
row counts come from a bincount with minlength = num_nodes, so nodes of
out-degree 0 keep their (empty) rows — the absorbing nodes the walks expect.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch


def to_csr(edge_index, num_nodes: Optional[int] = None, *, symmetrize: bool = False,
           dedup: bool = False, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(rowptr, col) int64 of a directed edge list, rows sorted by (row, col).

    Args:
        edge_index: int [2, E] (row, col) pairs; torch tensor or numpy array.
        num_nodes: node count V (default: max id + 1).
        symmetrize: add every reversed edge (undirected graphs).
        dedup: merge duplicate edges (the reference's pipeline keeps them).
        device: where to build (default: edge_index's device).
    """
    if isinstance(edge_index, np.ndarray):
        edge_index = torch.from_numpy(edge_index)
    if not isinstance(edge_index, torch.Tensor) or edge_index.dim() != 2 or edge_index.shape[0] != 2:
        raise ValueError("edge_index must be a [2, E] tensor or array")
    if device is not None:
        edge_index = edge_index.to(device)
    row = edge_index[0].to(torch.int64)
    col = edge_index[1].to(torch.int64)
    if symmetrize:
        row, col = torch.cat([row, col]), torch.cat([col, row])
    if num_nodes is None:
        num_nodes = int(torch.maximum(row.max(), col.max()).item()) + 1 if row.numel() else 0
    if row.numel() and (int(row.min().item()) < 0 or int(col.min().item()) < 0 or
                        int(row.max().item()) >= num_nodes or int(col.max().item()) >= num_nodes):
        raise ValueError("edge_index holds ids outside [0, num_nodes)")
    key = row * max(num_nodes, 1) + col
    key = torch.unique(key, sorted=True) if dedup else torch.sort(key).values
    r = torch.div(key, max(num_nodes, 1), rounding_mode="floor")
    c = key - r * max(num_nodes, 1)
    rowptr = torch.zeros(num_nodes + 1, dtype=torch.int64, device=row.device)
    torch.cumsum(torch.bincount(r, minlength=num_nodes), 0, out=rowptr[1:])
    return rowptr, c.contiguous()
