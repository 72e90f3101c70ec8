"""Test setup: import paths and the `gpu` marker.

`-m "not gpu"` runs on any machine (oracle pins, state logic, the C ABI's symbols and error paths). `-m gpu` runs the
parity tests proper on an MI355X, through the C ABI; on a machine without a ROCm GPU they are skipped.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "metal-inference-engine_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built librk_path.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def backend():
    """The ROCm backend on cuda:0 (raises, not skips, when the library is missing on a GPU machine)."""
    from backend.rocm import RocmBackend
    return RocmBackend("cuda:0")

