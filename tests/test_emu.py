"""The library's own kernels run on the CPU through the emulation in tests/emu/:
the .hip sources compiled for the host against a stand-in of the HIP runtime, a
block's threads as fibers, cross-lane operations as rendezvous of the wave's 64
lanes, loads into LDS landing only at the s_waitcnt that allows them, static and
dynamic LDS filled with stale bytes, every memory access under the address
sanitizer.  The emulation's lane models are pinned to a probe run on an MI355X
(fixtures/gfx950_lanes.bin); the kernels are then checked against the oracle as
the GPU tests check them, at small sizes.  CPU only."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "emu"))

pytestmark = pytest.mark.emu
CASES = str(HERE / "emu" / "cases.py")
# the cases that take a minute or more each run only with SBSA_EMU_LONG=1, so that
# the default CPU suite stays at a few minutes
long_case = pytest.mark.skipif(os.environ.get("SBSA_EMU_LONG", "0") != "1",
                               reason="long emulated case: set SBSA_EMU_LONG=1")


def _run(case, *args, **kw):
    import session
    rc, out = session.run(CASES, case, *map(str, args), **kw)
    assert rc == 0, f"{case}{args}: exit {rc}\n{out[-4000:]}"
    print(out.strip().splitlines()[-1])


def test_lane_models_match_the_gpu_probe(tmp_path):
    """The probe program through the emulation writes what it wrote on an MI355X:
    transposing LDS reads, both bf16 MFMA shapes (exact on these small-integer
    operands), v_permlane32_swap and the DPP controls."""
    import subprocess
    from build import build_program
    exe = build_program(HERE / "emu" / "probe_lanes.hip", tmp_path / "probe_lanes")
    out = tmp_path / "lanes.bin"
    subprocess.run([str(exe), str(out)], check=True, timeout=120)
    want = (HERE / "emu" / "fixtures" / "gfx950_lanes.bin").read_bytes()
    got = out.read_bytes()
    assert len(got) == len(want)
    assert got[:4096] == want[:4096], "operands differ"
    import numpy as np
    g = np.frombuffer(got[4096:], np.uint32)
    w = np.frombuffer(want[4096:], np.uint32)
    sections = {"ds_read_b64_tr_b16": (0, 512), "mfma_f32_32x32x16_bf16": (512, 1536),
                "mfma_f32_16x16x32_bf16": (1536, 1792), "v_permlane32_swap": (1792, 1920),
                "update_dpp": (1920, 2432)}
    for name, (a, b) in sections.items():
        assert np.array_equal(g[a:b], w[a:b]), f"{name}: {int((g[a:b] != w[a:b]).sum())} values differ"


def test_emulated_dense_prefix_chunk():
    _run("dense_chunk", 256, 8, 2, 128, 128, 191, 3)


@long_case
def test_emulated_sparse_chunk():
    _run("sparse_chunk", 1024, 8, 2, 128, 512, 767, 1, 2)


@long_case
def test_emulated_decode_steps():
    _run("decode_steps", 1024, 8, 2, 128, 5)


def test_emulated_decode_steps_in_several_rounds():
    # D = 256, G = 4 (192-row rounds), one prompt split and one suffix split and
    # a 512-token budget: each split takes its rows in two rounds
    _run("decode_steps", 1024, 4, 1, 256, 7, 1, 1, 512)


@long_case
def test_gpu_selection_and_append_tests_under_emulation():
    """The selection tests and the token-order append tests, run unchanged on the
    emulated kernels (each kernel's every memory access under the sanitizer)."""
    _run("gpu_tests", "test_gpu_select.py",
         "test_gpu_token_order.py::test_append_rows_bit_exact",
         "test_gpu_token_order.py::test_append_rows_flags_an_id_out_of_range", timeout=900)


@long_case
def test_kmeans_build_with_restarts_under_emulation():
    """The index build on keys that leave clusters empty (restarts drawn ahead and
    applied on the device, then on the host past two), run unchanged on the emulated
    kernels: assignment, member bitmaps, sums and centroid steps under the sanitizer."""
    _run("gpu_tests", "test_gpu_kmeans.py::test_build_with_empty_clusters_matches_the_oracle",
         timeout=900)
