"""pytest configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs everywhere (oracle, host logic, C-ABI loading and
validation); `-m gpu` needs an MI355X and calls the gfx950 kernels through
the C ABI.
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "diffusion-llm_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch.device("cuda:0")
