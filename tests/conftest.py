import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from tests._oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 (gfx950) once per session; fails loudly without one."""
    from woolly_amd import device

    print(f"[gpu] init device 0 pid={os.getpid()}", flush=True)
    device.init(0)
    print(f"[gpu] {device.device_name()}", flush=True)
    return device
