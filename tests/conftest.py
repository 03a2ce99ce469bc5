import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: larger CPU cases")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def ext():
    """The built HIP extension; on a GPU box a missing build is a failure, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nanotitan_amd.extension import get_hip_extension

    return get_hip_extension()


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work, so a run that dies mid-test says where.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield


GOLDEN = ROOT / "tests" / "golden"
os.environ.setdefault("PYTHONHASHSEED", "0")
