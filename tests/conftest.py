import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    """The GPU; a GPU test never silently skips when the card is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU (run with -m 'not gpu' on CPU)"
    import minitensor_amd as mt
    mt.lib()  # raises if libmtgemm.so was not built
    return torch.device("cuda:0")
