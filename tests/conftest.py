import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def hip_ready():
    """The HIP path must be live on a GPU box: no silent skip."""
    from tilegen_amd import runtime
    n = runtime.device_count()
    assert n >= 1, "no HIP device visible"
    info = runtime.device_info(0)
    print("\n[gpu] %s arch=%s cu=%d" % (info["name"], info["arch"], info["cu_count"]),
          flush=True)
    return info
