import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity against the CPU oracle")


@pytest.fixture(scope="session")
def hip_device():
    """The HIP device; a GPU test on a machine without one fails rather than skips."""
    import unpopped_amd as u

    n = u.device_count()
    if n < 1:
        pytest.fail("no HIP device visible: the gpu tests run on an MI355X")
    arch, cus = u.device_info()
    print(f"\n[gpu] device 0: {arch}, {cus} CUs", flush=True)
    return arch, cus
