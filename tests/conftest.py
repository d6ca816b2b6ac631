import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "pku-aiprogramming_amd")
OPT = os.path.join(PKG, "optimizer")
for p in (ROOT, PKG, OPT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP kernels")


def gpu_present() -> bool:
    return os.path.exists("/dev/kfd")


def pytest_collection_modifyitems(config, items):
    if gpu_present():
        return
    skip = pytest.mark.skip(reason="no GPU device node (/dev/kfd) in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
