import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def dsa():
    """The package, imported from tilelang-ascend_amd/ (the HIP library must be built)."""
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg.load_library()
    return pkg


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    return torch.device("cuda:0")
