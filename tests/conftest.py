"""Test configuration: the ``gpu`` marker and import paths."""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "semantic-block-sparse-attention_amd"
for p in (str(ROOT), str(PKG_DIR), str(ROOT / "tests" / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "emu: runs the HIP kernels on the CPU through tests/emu (slow)")
