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


# Achieved errors of the parity tests, printed at the end of the run so the
# margin to each tolerance is visible (test id, quantity, value, bar).
_ACHIEVED: list[tuple[str, str, float, float]] = []


@pytest.fixture
def record_error(request):
    """record_error(quantity, value, tolerance): keep the achieved error for
    the end-of-run summary and assert it is within the tolerance."""

    def record(quantity: str, value: float, tolerance: float) -> None:
        _ACHIEVED.append((request.node.name, quantity, float(value), float(tolerance)))
        assert value <= tolerance, f"{quantity}: {value:.4g} > {tolerance:.4g}"

    return record


def pytest_terminal_summary(terminalreporter):
    if not _ACHIEVED:
        return
    terminalreporter.section("achieved errors (value / tolerance)")
    worst: dict[str, tuple[float, float, str]] = {}
    for test, quantity, value, tol in _ACHIEVED:
        terminalreporter.write_line(f"{test:60s} {quantity:14s} {value:10.3e} / {tol:.1e}")
        if quantity not in worst or value / tol > worst[quantity][0] / worst[quantity][1]:
            worst[quantity] = (value, tol, test)
    for quantity, (value, tol, test) in sorted(worst.items()):
        terminalreporter.write_line(f"worst {quantity:14s} {value:10.3e} / {tol:.1e} ({100 * value / tol:.0f}% of the bar) in {test}")
