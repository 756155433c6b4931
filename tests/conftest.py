"""Test configuration.

`-m "not gpu"`: oracle pinning, host-side logic, C-ABI loading/exports.
`-m gpu`: parity of the HIP kernels (through the C ABI) against the oracle on
a ROCm GPU; skipped where no GPU is visible.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "kernel-pocs_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and runs the HIP kernels")
    config.addinivalue_line("markers", "slow: long-running case")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
