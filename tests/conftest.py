import os
import sys

import pytest

REPO_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO_DIR, "int8-transformer-kernels_amd")
for p in (REPO_DIR, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def capi():
    import int8k_capi

    return int8k_capi


@pytest.fixture(scope="session")
def ext():
    import torch  # noqa: F401  (the binding links against torch's libraries)
    import int8_ext

    return int8_ext


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")
