"""Shared pytest setup: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle-vs-golden checks, the host-side logic and the
C-ABI load/export checks on a CPU-only machine; `-m gpu` runs the parity tests
of the HIP path against the oracle on an MI355X.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gefen-x_amd")
for path in (ROOT, PKG):
    if path not in sys.path:
        sys.path.insert(0, path)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")
