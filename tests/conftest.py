import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE_ROOT = os.path.join(ROOT, "vllm-rlt_amd")
for path in (ROOT, PACKAGE_ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail loudly (not skip) when none is present."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible ROCm GPU"
    from vllm_rlt.kernels._hip import library

    library()  # ImportError here means the in-tree library was not built
    return torch.device("cuda:0")
