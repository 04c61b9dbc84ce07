"""Shared test setup: import paths, the ``gpu`` marker and GPU fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_DIR = ROOT / "ml-guided-program-search-for-shape-specialized-transformer-optimization_amd"
for path in (PACKAGE_DIR, ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library"
    )


@pytest.fixture(scope="session")
def gpu_device():
    """cuda:0 on a gfx950 box with the library loaded; never a silent skip
    when a GPU is present but the library is missing."""

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible to torch")
    from solution.kernels.hip import is_gfx950, load_library

    device = torch.device("cuda", 0)
    if not is_gfx950(device):
        pytest.skip(f"GPU is not gfx950: {torch.cuda.get_device_properties(0).gcnArchName}")
    load_library()  # raises HipLibraryError if the in-tree library is missing
    return device
