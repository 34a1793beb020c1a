import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through libpagoda_hip.so)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def dev():
    """The HIP device. GPU tests fail (never skip) when it cannot be opened:
    a silent skip would hide a missing native library."""
    from pagoda_amd import Device

    d = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    yield d
    d.sync()


@pytest.fixture(scope="session")
def ora():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle
