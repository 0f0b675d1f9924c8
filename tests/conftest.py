import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def gpu():
    """The product library on a live GPU. Fails loudly (never falls back) when it is missing."""
    import ninfer_amd
    from ninfer_amd import device

    ninfer_amd.lib()
    n = device.device_count()
    if n < 1:
        pytest.fail("no GPU visible to the ninfer_amd library")
    return device
