"""ctypes binding of libsbsa.so, the C ABI declared in include/sbsa.h.

The library is loaded from ``semblo_amd/_lib/libsbsa.so`` (built in-tree by
``build.py``).  There is no fallback: if the library is missing or a tensor
is not on a ROCm device, the call raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsbsa.so"

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# name -> (restype, argtypes), in the order of include/sbsa.h
SIGNATURES = {
    "sbsa_abi_version": (I32, []),
    "sbsa_route_vectors": (I32, [P, I64, I64, I32, I32, P, I64, P]),
    "sbsa_key_space": (I32, [P, I64, I64, I32, I32, P, P, P]),
    "sbsa_kmeans_assign": (I32, [P, I64, P, I64, P, I32, I32, P, P]),
    "sbsa_kmeans_update": (I32, [P, I64, P, I64, P, I32, I32, P, P, P, SZ, P]),
    "sbsa_kmeans_member_bits_bytes": (SZ, [I64, I32]),
    "sbsa_kmeans_iterate": (I32, [P, P, I64, P, I64, I32, I32, P, P, P, P, P, I32, P, P, P, P, SZ,
                                     I32, I32, P]),
    "sbsa_kmeans_centroids": (I32, [I32, P, P, P, P, I64, P, I32, I32, P, P, P]),
    "sbsa_bucket_layout_workspace_bytes": (SZ, [I64, I32]),
    "sbsa_bucket_layout": (I32, [P, I64, I32, I32, P, P, P, I64, P, P, P, SZ, P]),
    "sbsa_pack_kv": (I32, [P, P, I64, I64, I32, I32, P, I64, I64, P, P]),
    "sbsa_score_select": (I32, [P, I64, I64, P, P, P, I64, I64, I32, I32, I32, I32, I32, I32,
                                F32, F32, F32, I32, I32, P, P, P, P, P, P, P]),
    "sbsa_causal_sizes": (I32, [P, I64, P, P, I32, I32, I64, P, P]),
    "sbsa_reverse_index": (I32, [P, I32, I32, I32, P, P, P, P, P, I64, P, P]),
    "sbsa_prefill_items_bound": (I64, [I64, I32, I32, I32, I32]),
    "sbsa_prefill_items": (I32, [P, I32, I32, I32, I32, I32, P, P, P, P, I64, I64, P, P]),
    "sbsa_prefill_item_rows": (I32, []),
    "sbsa_prefill_attend": (I32, [P, I64, I64, I32, I32, I32, I32, P, I64, P, P, I64, I64, P, P,
                                  I32, P, P, P, P, P, P, P, I64, I64, P, I64, I64, F32, I32, P]),
    "sbsa_prefill_combine": (I32, [P, P, P, P, P, P, P, I64, I64, P, P, I64, I64, P, I32, I32,
                                   I32, I32, I32, P, P]),
    "sbsa_decode_workspace_bytes": (SZ, [I32, I32, I32, I32, I32, I32]),
    "sbsa_decode_step": (I32, [P, I64, P, I64, I32, P, P, I64, P, P, P, P, P, I64, P, I64, I32, P, I64,
                               I32, P, P, P, I32, I32, I32, I32, F32, F32, F32, I32, I32, F32, I32,
                               I32, P, SZ, P, I64, P, P, P]),
    "sbsa_decode_scratch_bytes": (SZ, []),
    "sbsa_decode_step_noalloc": (I32, [P, I64, P, I64, I32, P, P, I64, P, P, P, P, P, I64, P, I64,
                                       I32, P, I64, I32, P, P, P, I32, I32, I32, I32, F32, F32,
                                       F32, I32, I32, F32, I32, I32, P, I64, P, P, P]),
    "sbsa_nearest_cluster": (I32, [P, I64, I64, I64, I32, I32, I32, P, I32, P, P]),
    "sbsa_append_rows": (I32, [P, I64, I32, I32, P, P, P, P, P, P, P]),
    "sbsa_append_kv": (I32, [P, P, I64, I64, I64, I32, I32, P, I64, P, I64, P, I64, P, I64, P, P,
                             I32, P, P]),
    "sbsa_relayout_runs": (I32, [P, P, I64, I64, I64, I32, I32, P, I64, P, P, I32, P, I64, P, I64,
                                 P, I64, P]),
    "sbsa_gather_rows": (I32, [P, I64, I32, I32, P, I64, I64, I64, P, P, I64, I64, P]),
    "sbsa_repack_runs": (I32, [P, P, I64, I32, I32, I64, P, I64, P, P, I32, P, I64, P, I64, P]),
}

ERRORS = {1: "bad argument", 2: "unsupported shape", 3: "kernel launch failed",
          4: "buffer below its capacity bound"}

_LIB = None


def load() -> ctypes.CDLL:
    """Load libsbsa.so once; raise if it was not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("SBSA_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(
            f"libsbsa.so is not built ({path}); run "
            "`python semantic-block-sparse-attention_amd/build.py` (needs hipcc)")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def call(name: str, *args) -> int:
    """Call an entry point; raise RuntimeError on a nonzero status."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed: {ERRORS.get(rc, rc)}")
    return rc


def query(name: str, *args):
    """Call a size/bound query (no status code)."""
    return getattr(load(), name)(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor (None for a missing optional tensor)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError("libsbsa works on ROCm device tensors only; got a CPU tensor")
    return t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    """The current torch stream's hipStream_t."""
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the semblo_amd kernels run on the GPU only (no CPU fallback)")
