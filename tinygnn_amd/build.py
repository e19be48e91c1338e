"""Builds the libraries in-tree with hipcc.

* ``tinygnn_amd/_build/libtinygnn_amd.so`` -- the C-ABI (include/tinygnn_amd.h):
  every ``csrc/*.hip`` file compiled to an object under ``_build/obj`` (in
  parallel).  Device code is compiled for gfx950 only, with packed-fp32
  instructions disabled and floating-point contraction off, so that every
  fused multiply-add in the kernels is an explicit one.
* ``tinygnn_amd/_build/libtinygnn.so`` -- TinyGNN's C++ API
  (include/tinygnn/*.hpp) over the C-ABI, from ``cpp/*.cpp`` (host code).
* ``tinygnn_amd/_build/test_cpp_api`` -- the C++ API test (tests/cpp).
* ``tinygnn_amd/_build/test_throw_sites`` -- every throw statement of the
  reference driven through the C++ API (tests/cpp/throw_sites.cpp).
* ``tinygnn_amd/_build/test_numparse`` -- the CSV number conversions checked
  against the host C library (tests/cpp/test_numparse.cpp).

Usage: ``python -m tinygnn_amd.build [-j N] [--quiet]``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OBJ = os.path.join(BUILD, "obj")
LIB = os.path.join(BUILD, "libtinygnn_amd.so")
CPP = os.path.join(HERE, "cpp")
API_LIB = os.path.join(BUILD, "libtinygnn.so")
CPP_TEST = os.path.join(BUILD, "test_cpp_api")
THROW_TEST = os.path.join(BUILD, "test_throw_sites")
NUMPARSE_TEST = os.path.join(BUILD, "test_numparse")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
    "-ffp-contract=off",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
]


def _sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def _compile(src: str, quiet: bool) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC] + COMMON + DEVICE
    if src.endswith(".cpp"):
        cmd += ["-x", "hip"]
    cmd += ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if not quiet:
        msgs = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l]
        if msgs:
            print("\n".join(msgs), file=sys.stderr)
    return obj


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def _build_cpp_api() -> None:
    """The C++ API (include/tinygnn/*.hpp) as libtinygnn.so over the C-ABI
    library, and the C++ API test binary; host code only."""
    host = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{os.path.join(ROOT, 'include')}"]
    api_src = sorted(glob.glob(os.path.join(CPP, "*.cpp")))
    api_obj = []
    for s in api_src:
        o = os.path.join(OBJ, "api_" + os.path.basename(s) + ".o")
        _run(host + ["-c", s, "-o", o])
        api_obj.append(o)
    tmp = API_LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "-o", tmp] + api_obj +
         [f"-L{BUILD}", "-ltinygnn_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, API_LIB)
    test_src = os.path.join(ROOT, "tests", "cpp", "test_api.cpp")
    tmp = CPP_TEST + ".tmp"
    _run(host + [test_src, "-o", tmp, f"-L{BUILD}", "-ltinygnn", "-ltinygnn_amd",
                 "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, CPP_TEST)
    tmp = THROW_TEST + ".tmp"
    _run(host + [os.path.join(ROOT, "tests", "cpp", "throw_sites.cpp"), "-o", tmp,
                 f"-L{BUILD}", "-ltinygnn", "-ltinygnn_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, THROW_TEST)
    _build_pybind()
    # the CSV number conversions (csrc/numparse.hpp) compiled for the host and
    # checked against the C library in tests/test_numparse.py
    tmp = NUMPARSE_TEST + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-Wall", f"-I{CSRC}",
          os.path.join(ROOT, "tests", "cpp", "test_numparse.cpp"), "-o", tmp])
    os.replace(tmp, NUMPARSE_TEST)


def _build_pybind() -> None:
    """The Python module ``_tinygnn_core`` (pybind/tinygnn_core.cpp) over
    libtinygnn.so: the reference's binding surface, host code only."""
    import sysconfig

    import pybind11
    out = os.path.join(BUILD, "_tinygnn_core" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden", "-Wall",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{pybind11.get_include()}",
          f"-I{sysconfig.get_paths()['include']}",
          os.path.join(HERE, "pybind", "tinygnn_core.cpp"), "-o", tmp,
          f"-L{BUILD}", "-ltinygnn", "-ltinygnn_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)


def build(jobs: int | None = None, quiet: bool = True) -> str:
    """Compiles every source and links the shared libraries; returns the
    C-ABI library's path."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, quiet), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    _build_cpp_api()
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--quiet", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.quiet))


if __name__ == "__main__":
    main()
