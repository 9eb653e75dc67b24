import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "llm-mojo_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpkv's C ABI)")


@pytest.fixture(scope="session")
def gpu():
    """Every GPU test goes through here: fails (never skips) when no device is visible,
    so a GPU run cannot pass on a silent fallback."""
    from pkv import hip, lib

    n = hip.device_count()
    assert n > 0, "no HIP device visible"
    lib.load()
    return n
