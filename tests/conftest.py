import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    """The GPU every gpu-marked test runs on; a missing GPU is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test needs a GPU (run with -m 'not gpu' on a CPU host)")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # Print (and flush) what is about to run, so a run that ends the process
    # still names the case it was on.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
