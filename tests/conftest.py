import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


@pytest.fixture(scope="session")
def dev():
    """cuda:0, after checking the HIP library and a GPU are present (GPU tests fail loudly otherwise)."""
    import torch

    import scratchtape_amd

    scratchtape_amd.lib()  # raises if the library is not built
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")
