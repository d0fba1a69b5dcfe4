import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
os.environ.setdefault("TORCH_DEVICE_BACKEND_AUTOLOAD", "0")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from thintnpu_amd import capi
    capi.lib()
    return torch.device("cuda:0")


def seeded(seed: int):
    import torch
    g = torch.Generator().manual_seed(seed)
    return g
