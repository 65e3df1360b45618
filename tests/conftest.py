"""Test configuration: import paths and the `gpu` marker.

Tests marked ``gpu`` need an MI355X (ROCm GPU) and the built HIP library;
everything else runs on a CPU-only machine.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mini-ep_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
