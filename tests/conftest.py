import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
# helper modules next to the tests (qblocks)
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "slow: longer CPU or GPU case")


@pytest.fixture(scope="session")
def ctx():
    """One device context for the whole GPU session."""
    from llm_core_amd import hip

    if hip.device_count() < 1:
        pytest.fail("gpu test selected but no HIP device is visible")
    c = hip.Context(0)
    print(f"\n[axf] device: {c.device_name()}", flush=True)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a hang or fault is attributable
    if request.node.get_closest_marker("gpu"):
        print(f"\n[axf] start {request.node.nodeid}", flush=True)
    yield
