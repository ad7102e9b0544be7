"""pytest configuration: the `gpu` marker, import paths, shared helpers.

Tests marked `gpu` need an MI355X and call the HIP library through its C ABI;
everything else runs on the CPU (oracle pinning, host logic, ABI validation,
ISA contract of the built kernels)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "fp8-replayssm-gdn-kernel_amd"
for path in (REPO, PKG):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); calls the HIP kernels")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _no_wait_timeouts(request):
    """Every GPU test ends with the device's bounded-wait status word at zero:
    no decode workgroup gave up waiting for its coefficient chain."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    import gdnr_lib

    gdnr_lib.wait_timeouts(reset=True)
    yield
    assert gdnr_lib.wait_timeouts(reset=True) == 0, "a decode kernel's bounded wait gave up"


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-12))
