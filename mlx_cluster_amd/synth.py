"""Seeded synthetic graphs in CSR form for the benchmark configurations.

Not part of the walk path: these build the inputs the walks run on (the
reference's tests load Cora over the network instead,
/root/reference/tests/test_random_walk.py:18-28).  CSR here is always int64,
sorted by (row, col), with rowptr = [0, cumsum(bincount(row, minlength=V))],
so nodes of out-degree 0 keep their (empty) rows — unlike the reference
tests' np.unique-based rowptr, which drops them.

Generators run in torch on any device (GPU for the large configurations);
the small Cora-like graph is built with numpy.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np
import torch

from .csr import to_csr


def csr_from_edges(row: torch.Tensor, col: torch.Tensor, num_nodes: int, *,
                   symmetrize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Deduplicated CSR (rowptr, col) sorted by (row, col)."""
    return to_csr(torch.stack([row.to(torch.int64), col.to(torch.int64)]), num_nodes,
                  symmetrize=symmetrize, dedup=True)


def rmat_edges(scale: int, num_samples: int, a: float = 0.57, b: float = 0.19,
               c: float = 0.19, *, seed: int = 0, device="cpu"
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """R-MAT edge samples (Chakrabarti, Zhan, Faloutsos, SDM'04).

    Each sample picks one quadrant per level with probabilities (a, b, c,
    1-a-b-c); the row bit is set in quadrants c and d, the column bit in b
    and d.  Duplicates and self-loops are kept (csr_from_edges dedups).
    """
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    row = torch.zeros(num_samples, dtype=torch.int64, device=device)
    col = torch.zeros(num_samples, dtype=torch.int64, device=device)
    ab, abc = a + b, a + b + c
    for level in range(scale):
        u = torch.rand(num_samples, generator=g, device=device)
        bit = 1 << (scale - 1 - level)
        row_bit = u >= ab
        col_bit = ((u >= a) & (u < ab)) | (u >= abc)
        row |= row_bit.to(torch.int64) * bit
        col |= col_bit.to(torch.int64) * bit
        del u, row_bit, col_bit
    return row, col


def rmat_csr(scale: int, num_samples: int, *, seed: int = 0, device="cpu",
             symmetrize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    row, col = rmat_edges(scale, num_samples, seed=seed, device=device)
    return csr_from_edges(row, col, 1 << scale, symmetrize=symmetrize)


def ba_hub_csr(num_nodes: int, m: int, num_hubs: int, hub_degree: int, *, seed: int = 0,
               device="cpu") -> Tuple[torch.Tensor, torch.Tensor]:
    """Barabási–Albert-style graph plus injected hubs, symmetrized CSR.

    Node i >= 1 attaches to m targets j = floor(i * u^2), u ~ U[0,1): that is
    the expected preferential-attachment kernel of the BA model (a node born
    at time j has degree ~ m * sqrt(i / j) at time i, so P(j) ~ j^(-1/2)),
    drawn in parallel instead of sequentially.  Then num_hubs seeded hub ids
    each join hub_degree distinct random nodes.  Duplicates are merged.
    """
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.arange(1, num_nodes, dtype=torch.int64, device=device).repeat_interleave(m)
    u = torch.rand(src.numel(), generator=g, device=device, dtype=torch.float64)
    dst = torch.floor(src.to(torch.float64) * u * u).to(torch.int64)
    del u
    hubs = torch.randperm(num_nodes, generator=g, device=device)[:num_hubs]
    hub_src, hub_dst = [src], [dst]
    for h in hubs.tolist():
        nbrs = torch.randperm(num_nodes, generator=g, device=device)[:hub_degree]
        hub_src.append(torch.full_like(nbrs, h))
        hub_dst.append(nbrs)
    src = torch.cat(hub_src)
    dst = torch.cat(hub_dst)
    del hub_src, hub_dst
    return csr_from_edges(src, dst, num_nodes, symmetrize=True)


def cora_like(seed: int = 0, num_nodes: int = 2708, num_pairs: int = 5278
              ) -> Tuple[np.ndarray, np.ndarray]:
    """Preferential-attachment graph with Cora's size, symmetrized CSR (numpy).

    Every node i >= 1 attaches to m_i in {1, 2} distinct earlier nodes chosen
    with probability proportional to degree (sampling the endpoint list);
    the count of m_i = 1 nodes makes the total exactly num_pairs undirected
    pairs.  No self-loops or duplicates; every node has degree >= 1.
    """
    rng = np.random.default_rng(seed)
    n_single = 2 * (num_nodes - 1) - num_pairs
    if n_single < 1 or n_single > num_nodes - 1:
        raise ValueError("num_pairs not reachable with m in {1, 2}")
    single = set([1]) | set(rng.choice(np.arange(2, num_nodes), n_single - 1, replace=False).tolist())
    endpoints = [0]  # node 0 is the seed; the first attachment must hit it
    pairs = []
    for i in range(1, num_nodes):
        m = 1 if i in single else 2
        targets = set()
        while len(targets) < m:
            targets.add(int(endpoints[rng.integers(len(endpoints))]))
        for t in sorted(targets):
            pairs.append((t, i))
            endpoints.extend([t, i])
        if i == 1:
            endpoints.remove(0)  # drop the placeholder weight of the seed node
    pairs = np.asarray(pairs, dtype=np.int64)
    assert len(pairs) == num_pairs
    row = np.concatenate([pairs[:, 0], pairs[:, 1]])
    col = np.concatenate([pairs[:, 1], pairs[:, 0]])
    order = np.lexsort((col, row))
    row, col = row[order], col[order]
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.cumsum(np.bincount(row, minlength=num_nodes), out=rowptr[1:])
    return rowptr, col
