import os

# Every launcher that supports it verifies on the host, before launching,
# that its operands lie inside their device allocations (hai_common.h).
os.environ.setdefault("HAI_CHECK_BOUNDS", "1")

import pytest

from _hai import gpu_available


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to the HIP runtime")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
