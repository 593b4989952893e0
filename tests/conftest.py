"""pytest configuration: the `gpu` marker and shared fixtures.

CPU tests (`-m "not gpu"`) check the oracle against the reference's known
answers and closed forms, the host logic, and that the C ABI loads. GPU tests
(`-m gpu`) run the HIP kernels through the C ABI and compare with the oracle.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for _p in (ROOT, ROOT / "tests"):   # the package and oracle; the tests' helper modules
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def engine():
    """A janus context on cuda:0 bound to torch's current stream."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test collected without a GPU")
    from janus_amd.ops import ComputeEngine
    eng = ComputeEngine(0)
    yield eng
    eng.sync()
    eng.close()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O
