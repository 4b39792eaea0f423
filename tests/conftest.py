import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(autouse=True)
def _announce(request):
    """Print (and flush) the case name before each GPU test, so a run that dies on the
    GPU still names the case it was in."""
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield


def gpu_available() -> bool:
    if os.environ.get("FORGE_FORCE_NO_GPU") == "1":
        return False
    import torch

    return torch.cuda.is_available()
