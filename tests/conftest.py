import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("naiwa-rs_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 HIP device (MI355X)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, after checking a device is present (GPU tests only)."""
    import naiwa_moe

    if naiwa_moe.device_count() < 1:
        pytest.skip("no HIP device")
    info = naiwa_moe.device_info(0)
    print(f"[gpu] {info}", flush=True)
    return naiwa_moe
