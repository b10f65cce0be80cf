import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "cq-pretrain_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

os.environ.setdefault("TORCH_DEVICE_BACKEND_AUTOLOAD", "0")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def gpu_available():
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gdn():
    """The hip backend module, initialized on a GPU (tests marked gpu only)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU in this environment")
    from cqgdn import gated_delta_net

    gated_delta_net.initialize()
    return gated_delta_net
