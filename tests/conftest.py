import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "oxide-forge_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def rt():
    """One runtime for the whole GPU session (device 0)."""
    import oxforge

    print(f"[gpu] creating runtime on device 0", flush=True)
    r = oxforge.Runtime(0)
    yield r
    r.close()
