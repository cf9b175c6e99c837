"""Shared test setup: import paths, the `gpu` marker and common fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "soar.cpp_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs through libsoar_gn.so on the device)")


@pytest.fixture(scope="session")
def oracle():
    import soar_oracle
    soar_oracle.lib()
    return soar_oracle


@pytest.fixture(scope="session")
def gpu():
    """The loaded HIP library on a visible device (never a fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import soar_gn
    L = soar_gn.lib()  # raises SoarUnavailable if the library is missing
    assert L.soar_is_device_available() == 1
    return soar_gn
