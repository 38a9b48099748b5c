"""Shared test setup.

CPU tests (default, `-m "not gpu"`) pin the oracle (oracle/) against the reference built from
its sources and against closed-form checks, and check the C-ABI library's exports and struct
layouts without launching GPU work. GPU tests (`-m gpu`) run the HIP backend on cuda:0 and
compare it bit for bit with the oracle and the committed golden vectors.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def have_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def backend():
    """One HIP backend context for the GPU tests. The HIP library must be built: a missing
    library is an error, not a skip."""
    if not have_gpu():
        pytest.skip("no GPU in this environment")
    from hymt2_amd import lib
    b = lib.Backend()
    yield b
    b.close()


@pytest.fixture(scope="session")
def ref():
    """The reference library compiled from its sources (oracle/_ref), at the scalar ISA."""
    from oracle import refbind
    if not refbind.available():
        pytest.skip("oracle/_ref/libhymt2_ref.so not built (needs the reference tree)")
    refbind.set_isa("scalar")
    return refbind
