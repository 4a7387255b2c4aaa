import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    dev = torch.device("cuda", 0)
    name = torch.cuda.get_device_properties(dev).gcnArchName
    print(f"[gpu] device 0: {torch.cuda.get_device_name(dev)} arch={name}", flush=True)
    return dev


def pytest_runtest_logstart(nodeid, location):
    # Name the case before any GPU work so that a crash still shows which test ran.
    if os.environ.get("GW_TRACE_TESTS", "1") == "1":
        print(f"\n[start] {nodeid}", flush=True)
