import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "mimir-model_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmimg.so")


@pytest.fixture(scope="session")
def oracle():
    import mimref

    if not os.path.exists(mimref.LIB_PATH):
        mimref.build()
    mimref.lib()
    return mimref


@pytest.fixture(scope="session")
def gpu():
    """libmimg on device 0. Fails (does not skip) when the library or the GPU
    is missing: a GPU test must run the native path."""
    import mimg

    mimg.load()
    mimg.init(0)
    return mimg
