"""Build libsbsa_emu.so: the library's own .hip sources, rewritten by transform.py,
compiled for the host against the HIP stand-in, with the address sanitizer (every
plain memory access of the kernel code, and every load/store the emulation makes
for a buffer resource or a load into LDS, is checked).  Test infrastructure only.

    python tests/emu/build.py [--no-asan]
"""
from __future__ import annotations

import argparse
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
# SBSA_EMU_ROOT: another checkout whose sources to build (default: this one)
ROOT = Path(os.environ.get("SBSA_EMU_ROOT", HERE.parents[1])).resolve()
CSRC = ROOT / "semantic-block-sparse-attention_amd" / "csrc"
BUILD = HERE / "_build" if ROOT == HERE.parents[1] else ROOT / "tests" / "emu" / "_build_alt"
sys.path.insert(0, str(HERE))
from transform import transform  # noqa: E402


def clangxx() -> str:
    for cand in ("/opt/rocm/lib/llvm/bin/clang++", "clang++"):
        if os.path.exists(cand) or cand == "clang++":
            return cand
    raise RuntimeError("clang++ not found")


def asan_runtime() -> str:
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found")
    return hits[-1]


def build(asan: bool = True, jobs: int = 8) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    flags = ["-std=c++20", "-O2", "-g", "-fPIC", "-fno-omit-frame-pointer", "-Wno-unused-result",
             "-Wno-unknown-attributes", "-Wno-ignored-attributes",
             "-I", str(HERE / "include"), "-I", str(CSRC), "-I", str(ROOT / "include")]
    if asan:
        flags += ["-fsanitize=address", "-shared-libasan"]
    srcs = []
    for hip in sorted(CSRC.glob("*.hip")):
        cpp = BUILD / (hip.stem + ".cpp")
        text = transform(hip.read_text())
        if not cpp.exists() or cpp.read_text() != text:
            cpp.write_text(text)
        srcs.append(cpp)
    srcs.append(HERE / "emu_runtime.cpp")
    suffix = "asan" if asan else "plain"

    def compile_one(src: Path) -> Path:
        obj = BUILD / f"{src.stem}.{suffix}.o"
        deps = [src, HERE / "include" / "hip" / "hip_runtime.h", CSRC / "sbsa_common.h",
                ROOT / "include" / "sbsa.h"]
        if obj.exists() and obj.stat().st_mtime >= max(d.stat().st_mtime for d in deps):
            return obj
        cmd = [clangxx(), *flags, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode:
            raise RuntimeError(f"emulation build failed for {src.name}:\n{res.stderr[-6000:]}")
        return obj

    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    lib = BUILD / f"libsbsa_emu_{suffix}.so"
    cmd = [clangxx(), *flags, "-shared", "-o", str(lib), *map(str, objs), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"emulation link failed:\n{res.stderr[-4000:]}")
    return lib


def build_program(hip: Path, out: Path) -> Path:
    """A standalone .hip program (with its own main) through the emulation, no sanitizer."""
    BUILD.mkdir(parents=True, exist_ok=True)
    cpp = BUILD / (hip.stem + ".prog.cpp")
    cpp.write_text(transform(hip.read_text()))
    cmd = [clangxx(), "-std=c++20", "-O2", "-Wno-unknown-attributes", "-I", str(HERE / "include"),
           str(cpp), str(HERE / "emu_runtime.cpp"), "-o", str(out), "-lpthread", "-ldl"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"emulation build failed for {hip.name}:\n{res.stderr[-4000:]}")
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--no-asan", action="store_true")
    a = ap.parse_args()
    print(build(asan=not a.no_asan))
