import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _ensure_oracle_built():
    lib = os.path.join(ROOT, "oracle", "liboracle.so")
    src = os.path.join(ROOT, "oracle", "oracle.c")
    if not os.path.exists(lib) or os.path.getmtime(lib) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle_built()
    import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def device():
    """The GPU under test. Fails (does not skip) when none is usable: GPU
    tests run only where a GPU is expected."""
    from foundry_amd.device import HipDevice

    dev = HipDevice(0)
    print(f"[gpu] device: {dev.device_name()}", flush=True)
    yield dev
    dev.close()


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # flushed before every test so a run that ends the GPU box names its case
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
