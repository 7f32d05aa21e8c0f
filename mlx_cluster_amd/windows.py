"""Skip-gram context windows over walks (libmlxc.so: mlxc_context_windows,
mlxc_negative_windows).

The reference stops at the walks (/root/reference/random_walks/
BiasedRandomWalk.cpp:96).  Training node2vec embeddings on them next cuts
every walk into overlapping windows of context_size nodes, and draws
negative windows over random nodes; the layout here is torch_geometric's
Node2Vec.pos_sample / neg_sample: window-major, out[j * N + n] = walk n's
nodes j .. j + C - 1.
"""
from __future__ import annotations

import numbers
from typing import Optional

import numpy as np
import torch

from . import _lib
from .walks import (_as_tensor, _check_stream_arg, _enter_side_stream, _leave_side_stream, _on,
                    _on_cpu, _on_device, _out_type, _resolve_device, _side_stream,
                    _stream_handle)

_ELEM = {torch.int64: _lib.MLXC_OUT_INT64, torch.int32: _lib.MLXC_OUT_INT32}


def _int(x, name: str) -> int:
    if isinstance(x, bool) or not isinstance(x, numbers.Integral):
        raise TypeError(f"{name} must be an int")
    return int(x)


def context_windows(walks, context_size: int, *, stream=None) -> torch.Tensor:
    """Windows [W * N, C] of walks [N, L + 1], W = L + 2 - C, C = context_size.

    Row j * N + n holds walk n's nodes j .. j + C - 1 (torch_geometric
    Node2Vec.pos_sample order).  walks may be int64 or int32; the windows
    keep its dtype.  stream: as in random_walk ('cpu' runs the host twin).
    """
    _check_stream_arg(stream)
    if isinstance(walks, np.ndarray):
        walks = torch.from_numpy(walks)
    if not isinstance(walks, torch.Tensor) or walks.dim() != 2:
        raise ValueError("walks must be a 2-D [N, L + 1] tensor")
    if walks.dtype not in _ELEM:
        raise TypeError(f"walks must be int64 or int32, got {walks.dtype}")
    C = _int(context_size, "context_size")
    N, nodes = walks.shape
    if not 1 <= C <= min(32, nodes):
        raise ValueError("context_size must lie in [1, min(32, walk length + 1)]")
    W = nodes - C + 1
    lib = _lib.load()
    if _on_cpu(stream):
        walks = walks.cpu().contiguous()
        out = torch.empty((W * N, C), dtype=walks.dtype)
        rc = lib.mlxc_context_windows_cpu(walks.data_ptr() if N else None, N, nodes, C,
                                          _ELEM[walks.dtype], out.data_ptr() if N else None)
        _lib.check(rc, "context_windows")
        return out
    device = _resolve_device(stream, (walks,))
    handle = _stream_handle(stream, device)
    walks = _on(walks, device)
    out = torch.empty((W * N, C), dtype=walks.dtype, device=device)
    side = _side_stream(stream, device)
    _enter_side_stream(side, device)
    with _on_device(device):
        rc = lib.mlxc_context_windows(walks.data_ptr() if N else None, N, nodes, C,
                                      _ELEM[walks.dtype], out.data_ptr() if N else None, handle)
    _leave_side_stream(side, walks, out)
    _lib.check(rc, "context_windows")
    return out


def negative_windows(start, walk_length: int, context_size: int, num_nodes: int, *,
                     seed: Optional[int] = None, stream=None,
                     out_dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """Negative windows [W * N, C] (torch_geometric Node2Vec.neg_sample).

    The windows of the walks [start[n], u_1, ..., u_L], u_l drawn uniformly
    from [0, num_nodes) by Philox4x32-10 keyed by seed (counter (n, l)), so a
    seed gives the same windows on the GPU and with stream='cpu'.  seed=None
    draws one from torch's default CPU generator.
    """
    _check_stream_arg(stream)
    start = _as_tensor(start, torch.int64, "start").reshape(-1)
    L = _int(walk_length, "walk_length")
    C = _int(context_size, "context_size")
    V = _int(num_nodes, "num_nodes")
    if L < 0:
        raise ValueError("walk_length must be >= 0")
    if not 1 <= C <= min(32, L + 1):
        raise ValueError("context_size must lie in [1, min(32, walk_length + 1)]")
    out_type = _out_type(out_dtype)
    if seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    seed = int(seed) & (2**64 - 1)
    N = start.numel()
    W = L + 2 - C
    lib = _lib.load()
    if _on_cpu(stream):
        start = start.cpu().contiguous()
        out = torch.empty((W * N, C), dtype=out_dtype)
        rc = lib.mlxc_negative_windows_cpu(start.data_ptr() if N else None, N, L, C, V, seed,
                                           out_type, out.data_ptr() if N else None)
        _lib.check(rc, "negative_windows")
        return out
    device = _resolve_device(stream, (start,))
    handle = _stream_handle(stream, device)
    start = _on(start, device)
    out = torch.empty((W * N, C), dtype=out_dtype, device=device)
    side = _side_stream(stream, device)
    _enter_side_stream(side, device)
    with _on_device(device):
        rc = lib.mlxc_negative_windows(start.data_ptr() if N else None, N, L, C, V, seed,
                                       out_type, out.data_ptr() if N else None, handle)
    _leave_side_stream(side, start, out)
    _lib.check(rc, "negative_windows")
    return out
