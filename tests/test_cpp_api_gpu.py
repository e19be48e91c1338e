"""TinyGNN's C++ API (include/tinygnn/*.hpp over the C-ABI) on the GPU: runs
the C++ test program tests/cpp/test_api.cpp (built by tinygnn_amd.build into
tinygnn_amd/_build/test_cpp_api) -- the reference's known answers, error
contract, tensor coherence, Model vs layer-by-layer."""
import os
import subprocess

import pytest

from tinygnn_amd import build

pytestmark = pytest.mark.gpu


def test_cpp_api(gpu):
    assert os.path.exists(build.CPP_TEST), "C++ API test binary not built"
    r = subprocess.run([build.CPP_TEST], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout.splitlines()[-1]
