"""Shared test setup: import paths for the package root and the repo root, and the `gpu` marker."""

from __future__ import annotations

import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
PACKAGE = REPO / "moe-gemm-parallel-bench_amd"
for path in (str(PACKAGE), str(REPO)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmoegemm.so")
