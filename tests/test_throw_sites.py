"""Every throw statement of the reference's src/{tensor,ops,layers,model,
graph_loader}.cpp, driven through this build's C++ API (include/tinygnn/*.hpp
over libtinygnn.so), against the exception type and message the compiled
reference gives for the same call (tests/golden/throw_sites.tsv, written by
tests/golden/make_throw_sites.py from oracle/_ref/throw_sites_ref).

The driver (tests/cpp/throw_sites.cpp) is one source compiled against both
libraries.  On the CPU, the cases this build answers without a device run;
those that need one (the GraphLoader parses, which run on the device, the
device-side endpoint checks of edge_list_to_csr, and Model::load_weights,
whose layers hold their weights on the device) run in the GPU test.  Without
a device, those fail cleanly: TG_ERR_ALLOC / TG_ERR_HIP at the C-ABI and
std::runtime_error in the C++ API, with the HIP runtime's reason.
"""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "throw_sites.tsv")
OURS = os.path.join(ROOT, "tinygnn_amd", "_build", "test_throw_sites")
REF = os.path.join(ROOT, "oracle", "_ref", "throw_sites_ref")
REF_SRC = "/root/reference/src"
# graph_loader.cpp:142 ("empty line"): read_lines keeps only non-empty trimmed
# lines, on which the first getline always succeeds, so it cannot be reached.
UNREACHABLE = {"graph_loader.cpp:142"}


def run_driver(exe, mode):
    with tempfile.TemporaryDirectory() as tmp:
        os.mkdir(os.path.join(tmp, "d"))
        r = subprocess.run([exe, mode, "d"], cwd=tmp, capture_output=True, timeout=300)
        assert r.returncode == 0, (exe, r.returncode, r.stderr.decode(errors="replace"))
        return r.stdout.decode("utf-8")


def parse(text):
    cases = {}
    for line in text.splitlines():
        name, kind, msg = line.split("\t", 2)
        assert name not in cases, f"duplicate case {name}"
        cases[name] = (kind, msg)
    return cases


def expected():
    with open(FIXTURE, encoding="utf-8") as f:
        return parse(f.read())


def no_device():
    import torch
    return torch.cuda.device_count() == 0


def test_fixture_every_case_throws():
    for name, (kind, msg) in expected().items():
        assert kind in ("invalid_argument", "out_of_range", "runtime_error"), (name, kind)
        assert msg, name


def test_fixture_matches_compiled_reference():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/throw_sites_ref not built (needs the reference sources)")
    assert parse(run_driver(REF, "all")) == expected()


def test_every_throw_statement_has_a_case():
    """The cases name file:line of every `throw` in the reference's sources."""
    if not os.path.isdir(REF_SRC):
        pytest.skip("the reference's sources are not present")
    sites = set()
    for fn in ("tensor.cpp", "ops.cpp", "layers.cpp", "model.cpp", "graph_loader.cpp"):
        with open(os.path.join(REF_SRC, fn), encoding="utf-8") as f:
            for i, line in enumerate(f, 1):
                if re.search(r"\bthrow\s+std::", line):
                    sites.add(f"{fn}:{i}")
    covered = {name.split(" ", 1)[0] for name in expected()}
    assert sites - UNREACHABLE == covered - UNREACHABLE, (
        sorted(sites - covered - UNREACHABLE), sorted(covered - sites))
    assert len(sites) == 91


def test_host_cases_match_reference():
    """The cases answered without a device: same type, same text."""
    want = expected()
    got = parse(run_driver(OURS, "host"))
    assert len(got) >= 85, len(got)
    for name, v in got.items():
        assert v == want[name], (name, v, want[name])


def test_no_device_path():
    """Without a GPU: the cases that need one fail with a clean
    std::runtime_error naming the HIP runtime's reason, and the C-ABI returns
    TG_ERR_HIP (a kernel launch) or TG_ERR_ALLOC (an allocation), with the
    message, instead of crashing."""
    if not no_device():
        pytest.skip("a GPU is visible")
    want = expected()
    host = parse(run_driver(OURS, "host"))
    got = parse(run_driver(OURS, "all"))
    assert set(got) == set(want)
    device_cases = set(got) - set(host)
    assert device_cases
    for name in device_cases:
        kind, msg = got[name]
        assert kind == "runtime_error" and "no ROCm-capable device" in msg, (name, kind, msg)
    import tinygnn_amd as tg
    lib = tg.lib
    lib.load()
    p = ctypes.c_void_p(0x1000)  # never dereferenced: every call fails first
    assert lib.tg_relu(16, p, None) == 4  # TG_ERR_HIP
    assert b"no ROCm-capable device" in lib.tg_last_error()
    assert lib.tg_spmm(10, 10, 4, 10, p, p, p, p, 4, p, 4, None) == 5  # TG_ERR_ALLOC
    assert b"no ROCm-capable device" in lib.tg_last_error()


@pytest.mark.gpu
def test_all_cases_match_reference():
    """Every case, the device ones included (the parses, the endpoint checks
    and load_weights run on the GPU): same type, same text."""
    want = expected()
    got = parse(run_driver(OURS, "all"))
    assert set(got) == set(want)
    for name, v in got.items():
        assert v == want[name], (name, v, want[name])
