"""Pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` call the HIP kernels through the C ABI and need a ROCm device;
everything else runs on the CPU (oracle pinning, host-side API, library symbols).
"""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); calls the HIP kernels")
