"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X and the built library; everything else
runs on the CPU (oracle pinning, host logic, ABI loading).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: full-size (benchmark configuration) cases")


def pytest_sessionstart(session):
    """Builds the C oracle and the HIP library when they are missing and the
    compilers are present (a fresh checkout); the GPU box receives both
    prebuilt and never compiles here."""
    import shutil
    import subprocess
    oracle_so = os.path.join(ROOT, "oracle", "_build", "libtgoracle.so")
    if not os.path.exists(oracle_so) and shutil.which("gcc") and shutil.which("make"):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "oracle"], check=True)
    from tinygnn_amd import _lib
    if not os.path.exists(_lib.LIB_PATH) and os.path.exists("/opt/rocm/bin/hipcc"):
        from tinygnn_amd import build
        build.build()


@pytest.fixture(scope="session")
def restate():
    import oracle
    return oracle.restate()


@pytest.fixture(scope="session")
def reference():
    import oracle
    if not oracle.has_reference():
        pytest.skip("oracle/_ref/libtgref.so not built (needs the reference sources)")
    return oracle.reference()


@pytest.fixture(scope="session")
def gpu():
    """The torch module, after checking that a GPU is present (fails loudly
    instead of skipping: a GPU test must never pass without a GPU)."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    torch.cuda.init()
    return torch
