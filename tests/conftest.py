import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs the HIP library")


@pytest.fixture(scope="session")
def device():
    """The gfx950 device. GPU tests fail (never skip) when none is present: they only run
    with -m gpu, on a GPU host."""
    import l0llm_amd as l0

    if not l0.runtime_is_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    dev = l0.Device(0)
    print(f"\n[device] {dev.name}, {dev.compute_units} CUs", flush=True)
    yield dev
    dev.close()


@pytest.fixture(scope="session")
def suite(device):
    import l0llm_amd as l0

    return l0.LlmKernelSuite(device)


@pytest.fixture(autouse=True)
def _announce(request):
    # Names the running case before any GPU work, so a lost box still shows where it was.
    if request.node.get_closest_marker("gpu"):
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield


os.environ.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))
