"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` tests run anywhere (oracle, host logic, C-ABI export checks);
``-m gpu`` tests need an MI355X and call the HIP kernels through the C-ABI.
"""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "kimi-k3-mlx-macmini_amd"
for p in (ROOT, PKG_DIR):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libk3hip.so")
