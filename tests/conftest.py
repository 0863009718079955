import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP backend on the device)")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    # The library must load either way (a missing build is an error, not a skip);
    # only the absence of a device skips the device tests.
    from lokal_amd import _lib
    if _lib.lib().lkhip_device_count() == 0:
        skip = pytest.mark.skip(reason="no HIP device visible")
        for it in gpu_items:
            it.add_marker(skip)
