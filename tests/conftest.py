"""pytest configuration.

Markers: ``gpu`` — needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU. GPU tests call the HIP kernels through the C ABI (``cuda_amd``) and
fail — never silently fall back — if the library is missing.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)

torch = pytest.importorskip("torch")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an AMD Instinct GPU (gfx950)")


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.fixture(scope="session")
def dev():
    """The GPU device; GPU tests are skipped (not failed) without one, as in
    the reference's conftest (tests/conftest.py:20-28 there)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    import cuda_amd._lib as lib
    lib.load()  # raises if the HIP library was not built
    return torch.device("cuda:0")
