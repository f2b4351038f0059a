import os
import sys

import pytest

# torch first: its wheel carries its own HIP runtime, and the native
# libraries (libsi_amd.so, libsi_host.so) must bind to that copy.  Loaded
# before torch, they would bring the system runtime and the two would
# compete for the device (whichever initializes second fails).
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "simple-inference_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C-ABI on cuda:0)")
    config.addinivalue_line("markers", "slow: long CPU case")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle_py import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle_py import Reference, have_reference
    if not have_reference():
        pytest.skip("oracle/_ref not built (reference sources absent on this host)")
    return Reference()


@pytest.fixture(autouse=True)
def _release_device_tensors():
    yield
    import sys
    h = sys.modules.get("tests.gpu_helpers")
    if h is not None:
        h.KEEP.clear()
