import os
import sys

import pytest

# torch first: its bundled HIP runtime must be the process's one before
# libmagnetar_gpu.so (linked against the same soname) is loaded, or torch
# later finds no device
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "magnetar-provider-cpu_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ctx():
    import magnetar_gpu

    c = magnetar_gpu.Context(0)
    yield c
    c.close()
