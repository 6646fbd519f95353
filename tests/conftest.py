import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def lib():
    from credit_amd import hip_lib

    if not hip_lib.LIB_PATH.is_file():
        import __graft_entry__

        __graft_entry__.build()
    return hip_lib.load_library()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test scheduled without a visible GPU")
    return torch.device("cuda:0")
