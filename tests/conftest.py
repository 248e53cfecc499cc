"""Test configuration: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X and the built libqvp.so; everything else runs
on the CPU (`pytest -m "not gpu"`).
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for sub in ("qwenvl-paged_amd", "oracle", "tests"):
    p = str(ROOT / sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
