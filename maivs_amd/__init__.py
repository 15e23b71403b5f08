"""maivs_amd: MI355X-native batched cell-major search for the MAIVS FlatCellIndex.

``FlatCellIndex`` keeps the reference's Python API (``maivs.FlatCellIndex``,
src/index.rs:2670-3603): build on the host (train_centroids -> add_batch -> compact), then
``search_batch(queries, k, nprobe, target_confidence, beta, cell_major=True)`` runs on the GPU
through libmaivs_gpu.so's C ABI. There is no CPU search path: when the GPU library or the
configuration is missing, search_batch raises.
"""
from __future__ import annotations

import os

_HERE = os.path.dirname(os.path.abspath(__file__))

try:
    from ._maivs import FlatCellIndex  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(f"maivs_amd native module is not built ({e}); run python -m maivs_amd.build") from e

__all__ = ["FlatCellIndex", "preset"]


def preset(dim: int, n: int, profile: str = "quality") -> FlatCellIndex:
    """An unbuilt index configured like the reference's published presets
    (bench/fair/fairbench.py:98-106); the caller trains with max(16, n // 128) cells."""
    ix = FlatCellIndex(dim, "binary", 32, 0x5EED, 0)
    if profile == "memory":
        ix.set_per_dim_sq(True)
    elif profile != "quality":
        raise ValueError(f"unknown profile {profile!r}")
    ix.set_orthogonal_polysemy(2, 1.0)
    ix.set_fastscan(True)
    ix.set_two_stage(True, 2)
    ix.set_graph_route(False, 10 ** 9)
    ix.set_tree_route(True, 2048, 16)
    ix.set_adaptive(True, 0.02)
    return ix


def build_preset(base, profile: str = "quality", ids=None, gpu_build: bool = False) -> FlatCellIndex:
    """train_centroids(base, max(16, n // 128)) -> add_batch -> compact, as the reference's bench.
    gpu_build runs the build's k-means and placement on the GPU (bit-identical index)."""
    import numpy as np

    n = len(base)
    ix = preset(base.shape[1], n, profile)
    ix.set_gpu_build(gpu_build)
    ix.train_centroids(base, max(16, n // 128))
    ix.add_batch(list(range(n)) if ids is None else list(ids), np.ascontiguousarray(base, np.float32))
    ix.compact()
    return ix
