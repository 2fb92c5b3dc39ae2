"""The C ABI: the library loads (no GPU needed) and exports what include/sbsa.h declares,
with the argument counts the ctypes binding uses."""
from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sbsa.h"


def _declarations():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(int|size_t|int64_t)\s+(sbsa_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in m.group(3).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(2)] = len(args)
    return decls


def test_header_declares_the_entry_points():
    decls = _declarations()
    for name in ("sbsa_score_select", "sbsa_prefill_attend", "sbsa_decode_step",
                 "sbsa_kmeans_assign", "sbsa_bucket_layout", "sbsa_reverse_index"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    lib = _lib.load()
    decls = _declarations()
    for name in decls:
        assert hasattr(lib, name), name
    for name, n in decls.items():
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        assert len(_lib.SIGNATURES[name][1]) == n, f"{name}: header {n} args, binding {len(_lib.SIGNATURES[name][1])}"
    assert lib.sbsa_abi_version() == 4


def test_size_queries_run_without_a_gpu():
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    n = _lib.query("sbsa_decode_workspace_bytes", 16, 4, 128, 256, 64, 8)
    assert n >= 16 * 72 * 256 * 4
    assert _lib.query("sbsa_prefill_items_bound", 1000, 8192, 4, 128, 32) >= 1000 // 32
    assert _lib.query("sbsa_bucket_layout_workspace_bytes", 131072, 128) >= 128 * 128 * 4


def test_product_path_refuses_cpu_tensors():
    import torch
    from semblo_amd import _lib
    from semblo_amd.trivial_router import trivial_router_vectors
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    with pytest.raises(RuntimeError):
        trivial_router_vectors(torch.randn(4, 2, 64).to(torch.bfloat16))


def test_entry_points_reject_bad_arguments_before_any_launch():
    """Argument checks return SBSA_ERR_ARG (1) before any launch, so they run
    here without a GPU (the pointers below are never dereferenced)."""
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    lib = _lib.load()
    p = 256                                   # stand-in for a device pointer
    # k-means iterations it0..it1 with it1 < it0
    assert lib.sbsa_kmeans_iterate(p, p, 256, p, 100, 64, 256, p, p, p, p, None, 0, None, p, p, p,
                                   1 << 20, 3, 2, None) == 1
    # restart rows without their flags, and with no draws
    assert lib.sbsa_kmeans_iterate(p, p, 256, p, 100, 64, 256, p, p, p, None, p, 2, None, p, p, p,
                                   1 << 20, 0, 2, None) == 1
    assert lib.sbsa_kmeans_iterate(p, p, 256, p, 100, 64, 256, p, p, p, None, p, 0, p, p, p, p,
                                   1 << 20, 0, 2, None) == 1
    # the update's member bitmaps smaller than the bound
    need = lib.sbsa_kmeans_member_bits_bytes(1000, 64)
    assert need == 64 * 32 * 4
    assert lib.sbsa_kmeans_update(p, 256, p, 1000, p, 64, 256, p, p, p, need - 1, None) == 4
    # the work list without the reverse index's arrays
    assert lib.sbsa_prefill_items(p, 4, 64, 128, 32, 1, None, p, p, p, 100, 0, p, None) == 1
    # a window that starts after the chunk
    assert lib.sbsa_prefill_attend(p, 4096, 256, 128, 16, 4, 256, p, 1024, p, p, 1024, 256, p, p,
                                   64, p, p, p, p, p, p, p, 4096, 256, p, 512, 1024, 0.0625, 0,
                                   None) == 1


def test_attend_refuses_windows_past_the_32bit_buffer_range():
    """A window whose rows span 4 GiB or more (here a fused-QKV row stride of 12,288 and
    200,000 positions) cannot be addressed by the tile loads' buffer resources: the entry
    point refuses it (SBSA_ERR_UNSUPPORTED) instead of reading zeros past the wrap."""
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    lib = _lib.load()
    p = 256
    args = [p, 4096, 256, 128, 16, 4, 256, None, 0, p, p, 12288, 256, None, None, 32, None,
            None, p, p, None, None, p, 4096, 256, None, 200000, 0, 0.0625, 0, None]
    assert lib.sbsa_prefill_attend(*args) == 2


def test_combine_refuses_rows_that_are_not_16_byte_aligned():
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    lib = _lib.load()
    p = 256
    # G * D = 1024: 16-byte row pieces; an output row stride of 4 elements is refused
    assert lib.sbsa_prefill_combine(p, p, p, p, p, p, p, 4096, 256, p, p, 4, 256, None,
                                    8, 16, 4, 256, 128, None, None) == 1
    assert lib.sbsa_prefill_combine(p, p, p, p, p, p, p, 4100, 256, p, p, 4096, 256, None,
                                    8, 16, 4, 256, 128, None, None) == 1


def test_decode_without_allocation_refuses_shapes_past_its_scratch():
    """sbsa_decode_step_noalloc returns SBSA_ERR_CAPACITY (4) before any GPU call when the
    step's scratch would pass the library's static array."""
    from semblo_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libsbsa.so is not built here")
    lib = _lib.load()
    p = 256
    cap = lib.sbsa_decode_scratch_bytes()
    assert cap == 8 << 20
    # 64 query heads x 500 splits x 256 dims of fp32 partials: far past 8 MiB
    assert _lib.query("sbsa_decode_workspace_bytes", 64, 8, 1024, 256, 492, 8) > cap
    assert lib.sbsa_decode_step_noalloc(p, 256, p, 256, 1, None, None, 0, p, p, p, p, p, 1000, p,
                                        4, 256, p, 1000, 4, None, None, None, 64, 8, 1024, 256,
                                        10.0, 0.25, 100.0,
                                        16, 0, 0.0625, 492, 8, p, 256, None, None, None) == 4
