import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmixmoe on the device)")


@pytest.fixture(scope="session")
def gpu_lib():
    from mixlab_amd import _lib

    return _lib.init()
