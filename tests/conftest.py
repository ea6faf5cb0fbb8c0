import os
import sys

import pytest

# torch bundles its own HIP runtime (libamdhip64.so, SONAME libamdhip64.so.7).
# Imported first, that runtime is the process's only one: libane_hip.so's
# libamdhip64.so.7 then resolves to it.  Were libane_hip.so loaded first, the
# later torch import would load a second runtime (it asks for libamdhip64.so),
# and torch's device calls in the tests that use its tensors as plain device
# memory fail ("No HIP GPUs are available").  So torch is imported before any
# test can load the library, whatever subset of tests runs.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "autoresearch-go-ane_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")
    config.addinivalue_line("markers", "slow: long CPU test")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import ane
    return ane
