"""pytest configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the CPU suite (oracle pinning, host-side contracts,
C-ABI library load/export checks).  ``-m gpu`` runs the parity tests proper on
a ROCm GPU, through the C-ABI library.
"""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "bdh-gpu-fast_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a ROCm GPU and the built HIP library (parity tests)"
    )
