import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded (GPU tests only)."""
    import torch

    assert torch.cuda.is_available(), "GPU test selected but no ROCm device is visible"
    import toyinfer_amd.attn  # noqa: F401  (fails loudly if the .so is missing)

    return torch.device("cuda:0")
