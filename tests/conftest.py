import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("qwen-omni-inference-rs_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs through liblq8.so)")


@pytest.fixture(scope="session")
def ctx():
    import lq8

    c = lq8.Context(0)
    yield c
    c.close()
