import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libtiler_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One bound context for the whole GPU session (one process, one device)."""
    import tiler_amd

    c = tiler_amd.Context(0)
    print(f"\n[tiler-hip] bound {c.environment['device_name']} {c.environment['gcn_arch_name']} "
          f"CUs={c.environment['compute_units']}", flush=True)
    yield c
    c.close()
