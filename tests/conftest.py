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


#: Prefixes of the lines a parity test prints about its agreement with the
#: oracle (teacher-forced pick counts, logit-error spreads, free-run
#: divergence); the run's summary repeats them so the counts appear in the tail
#: of the output even when pytest captures each test's own output.
_RECORD_PREFIXES = ("[agreement]", "[spread]", "[free run]", "[exact]")
_records: list[str] = []


def pytest_runtest_logreport(report):
    if report.when != "call":
        return
    for _, text in report.sections:
        for line in text.splitlines():
            if line.startswith(_RECORD_PREFIXES):
                _records.append(f"{report.nodeid.split('::')[-1]}: {line}")


def pytest_terminal_summary(terminalreporter):
    if _records:
        terminalreporter.section("oracle agreement records")
        for line in _records:
            terminalreporter.write_line(line)
