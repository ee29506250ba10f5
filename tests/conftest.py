"""Shared pytest configuration.

`-m gpu` tests need an MI355X (gfx950) and call libdmc_hip through its C ABI;
everything else runs on the CPU (oracle pins, golden vectors, host logic, ABI
export checks).
"""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def hip():
    """The product package with its device confirmed; a GPU test without a
    usable device fails (it never falls back)."""
    import demonic_amd as d
    assert d.available(), "libdmc_hip reports no usable gfx950 device: " + \
        d._lib.load().dmc_hip_last_error().decode()
    return d
