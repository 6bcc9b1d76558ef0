import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "llm-shield_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: full-size model cases")


def gpu_available() -> bool:
    """True when the HIP runtime sees a device (checked without initialising torch)."""
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no GPU in this container")
    import jev  # noqa: F401  -- raises if libjev is not built
    jev.lib()
    return True
