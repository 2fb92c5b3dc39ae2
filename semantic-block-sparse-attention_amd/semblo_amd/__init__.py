"""semblo_amd: the MI355X-native semantic block-sparse attention path.

A drop-in for pfnet-research/semantic-block-sparse-attention's sparse
attention core (block build, centroid selection, KV-outer sparse prefill and
the graph-capturable sparse decode step), with every array operation in
hand-written gfx950 HIP kernels behind the C ABI of include/sbsa.h.
"""
from __future__ import annotations

from . import _lib
from .config import SembloRuntimeConfig, num_flat_clusters

__all__ = ["SembloRuntimeConfig", "num_flat_clusters", "load_library"]


def load_library():
    """Load libsbsa.so (raises if it is not built)."""
    return _lib.load()
