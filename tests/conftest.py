import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")


def gpu_visible():
    """True when a HIP device is visible (checked without initialising HIP in this process)."""
    if os.environ.get("HIP_VISIBLE_DEVICES", None) == "":
        return False
    return Path("/dev/kfd").exists() and any(Path("/dev/dri").glob("renderD*"))


@pytest.fixture(scope="session")
def eng():
    """The library's Engine; GPU tests need the built .so and fail loudly without it."""
    import ijah_amd
    return ijah_amd.load_engine()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O
