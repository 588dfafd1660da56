import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels through the C ABI")


@pytest.fixture(scope="session")
def ctx():
    """An open C-ABI context on cuda:0 (gpu tests only)."""
    import torch  # noqa: F401  (initialises the HIP runtime for tensor allocation)
    import dyninfer_amd as d

    c = d.Context(0)
    yield c
    c.close()
