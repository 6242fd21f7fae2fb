"""Test configuration.

``gpu``-marked tests run the HIP kernels and compare them with the NumPy
oracle under ``oracle/``; the rest run on any host (oracle pinning, the
Python boundary, the C-ABI exports).
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """Initialise the library on the GPU.  A missing library or a failing
    initialisation is an error, not a skip: GPU tests must run the HIP path."""
    from enilnets_amd import _lib
    _lib.lib()
    info = _lib.device_info()
    print(f"\n[gpu] {info.name.decode()} {info.arch.decode()} CUs={info.compute_units}",
          flush=True)
    return info
