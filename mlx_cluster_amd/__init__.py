"""MI355X-native random-walk path of vinayhpandya/mlx_cluster.

Drop-in for the reference package's two functions (re-exported by
/root/reference/mlx_cluster/__init__.py:3-4):

    import mlx_cluster_amd as mlx_cluster
    walks = mlx_cluster.random_walk(rowptr, col, start, rand, walk_length)
    walks = mlx_cluster.rejection_sampling(rowptr, col, start, walk_length, p, q)

The walks run in hand-written HIP kernels for gfx950 (libmlxc.so, C ABI in
include/mlxc.h); the package has no CPU fallback.
"""
from .csr import to_csr
from .walks import csr_check, philox_uniform, random_walk, rejection_sampling
from .windows import context_windows, negative_windows

__all__ = ["random_walk", "rejection_sampling", "csr_check", "philox_uniform", "to_csr",
           "context_windows", "negative_windows"]
__version__ = "0.1.0"
