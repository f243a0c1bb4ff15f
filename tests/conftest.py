import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libkvhip.so")


@pytest.fixture(scope="session")
def hip_device():
    """The first HIP device; fails (not skips) when a gpu-marked test runs without one."""
    import torch

    from kvserve_amd import hip_available

    assert torch.cuda.is_available(), "gpu test selected but no GPU is visible"
    assert hip_available(), "gpu test selected but libkvhip.so did not load"
    return torch.device("cuda:0")
