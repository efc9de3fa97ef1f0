import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _flush_print(msg):
    print(msg, flush=True)


@pytest.fixture(scope="session")
def device():
    import frizzle_amd
    dev = frizzle_amd.Device(0)
    yield dev
    dev.close()


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # Print which case runs before it touches the GPU, so a crash names it.
    if request.node.get_closest_marker("gpu"):
        _flush_print(f"\n[gpu case] {request.node.nodeid}")
    yield
