"""Run libsbsa's host code on CPU tensors against the emulated library.

``activate()`` points ``semblo_amd._lib`` at tests/emu/_build/libsbsa_emu_*.so and
lets its pointer and stream helpers take CPU tensors, in this process only (the
product's helpers refuse CPU tensors).  ``run(case_module, case, *args)`` runs a
case function in a child Python with the address sanitizer's runtime preloaded
(required to load the sanitized library) and returns its exit status and output.
Test infrastructure only.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
# SBSA_EMU_ROOT: another checkout whose library and host code to run (default: this one)
ROOT = Path(os.environ.get("SBSA_EMU_ROOT", HERE.parents[1])).resolve()
PKG = ROOT / "semantic-block-sparse-attention_amd"


def library(asan: bool = True) -> Path:
    sys.path.insert(0, str(HERE))
    from build import build
    return build(asan=asan)


class _Stream:
    """A host stand-in for a torch.cuda.Stream (work runs in issue order anyway)."""
    cuda_stream = 0

    def __init__(self, *a, **k):
        pass

    def wait_event(self, *a):
        pass

    def wait_stream(self, *a):
        pass

    def synchronize(self):
        pass

    def record_event(self, ev=None):
        return ev or _Event()


class _Event:
    def __init__(self, *a, **k):
        pass

    def record(self, *a):
        pass

    def synchronize(self):
        pass

    def wait(self, *a):
        pass

    def query(self):
        return True

    def elapsed_time(self, other):
        return 0.0


def _host_cuda_surface() -> None:
    """The few torch.cuda calls of the host code, as host no-ops (this process only)."""
    import contextlib
    import torch
    empty = torch.empty

    def empty_unpinned(*a, **k):
        k.pop("pin_memory", None)
        return empty(*a, **k)

    zeros = torch.zeros

    def zeros_unpinned(*a, **k):
        k.pop("pin_memory", None)
        return zeros(*a, **k)

    torch.empty = empty_unpinned
    torch.zeros = zeros_unpinned
    torch.Tensor.pin_memory = lambda self, *a, **k: self
    torch.cuda.Event = _Event
    torch.cuda.Stream = _Stream
    torch.cuda.current_stream = lambda *a, **k: _Stream()
    torch.cuda.stream = lambda *a, **k: contextlib.nullcontext()
    torch.cuda.synchronize = lambda *a, **k: None
    torch.Tensor.record_stream = lambda self, *a: None


def activate(lib_path: str | os.PathLike) -> None:
    sys.path.insert(0, str(PKG))
    sys.path.insert(0, str(ROOT))
    _host_cuda_surface()
    from semblo_amd import _lib
    lib = ctypes.CDLL(str(lib_path))
    for name, (res, args) in _lib.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib._LIB = lib
    _lib.ptr = lambda t: None if t is None else t.data_ptr()
    _lib.stream = lambda device=None: 0
    _lib.require_device = lambda *t: None


def run(case_file: str, case: str, *args: str, asan: bool = True, timeout: int = 900,
        extra_env: dict | None = None):
    """Run ``case(*args)`` of the module at ``case_file`` in a child process against
    the emulated library; returns (returncode, combined output)."""
    from build import asan_runtime
    lib = library(asan)
    env = dict(os.environ)
    if asan:
        env["LD_PRELOAD"] = asan_runtime()
        env["ASAN_OPTIONS"] = "detect_leaks=0:verify_asan_link_order=0:abort_on_error=1"
    env["SBSA_EMU_LIB"] = str(lib)
    env["OMP_NUM_THREADS"] = "1"
    env.update(extra_env or {})
    code = (f"import sys; sys.path.insert(0, {str(HERE)!r}); import session; "
            f"session.activate({str(lib)!r}); import runpy; "
            f"mod = runpy.run_path({case_file!r}); mod[{case!r}](*{list(args)!r})")
    import tempfile
    with tempfile.TemporaryFile(mode="w+") as log:
        proc = subprocess.Popen([sys.executable, "-c", code], env=env, stdout=log,
                                stderr=subprocess.STDOUT, text=True)
        try:
            rc = proc.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            proc.kill()
            proc.wait()
            rc = -9
        log.seek(0)
        return rc, log.read()
