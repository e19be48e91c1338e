#!/usr/bin/env python3
"""Writes tests/golden/throw_sites.tsv: the exception type and message of
every throw statement of the reference's src/{tensor,ops,layers,model,
graph_loader}.cpp, as the REAL reference reports them.

The driver is tests/cpp/throw_sites.cpp compiled against the reference's own
sources by oracle/Makefile (oracle/_ref/throw_sites_ref; development
container only).  It is run in mode "all" from a scratch directory with the
relative file directory "d", the same invocation tests/test_throw_sites.py
uses for this build's driver, so file names in the messages agree.

Usage: python tests/golden/make_throw_sites.py
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_DRIVER = os.path.join(ROOT, "oracle", "_ref", "throw_sites_ref")
OUT = os.path.join(HERE, "throw_sites.tsv")


def run_driver(exe: str, mode: str = "all") -> str:
    """The driver's output, run from a fresh scratch directory."""
    with tempfile.TemporaryDirectory() as tmp:
        os.mkdir(os.path.join(tmp, "d"))
        r = subprocess.run([exe, mode, "d"], cwd=tmp, capture_output=True, timeout=120)
        if r.returncode != 0:
            raise RuntimeError(f"{exe} exited {r.returncode}: {r.stderr.decode()}")
        return r.stdout.decode("utf-8")


def main() -> None:
    if not os.path.exists(REF_DRIVER):
        sys.exit(f"{REF_DRIVER} is missing: run make -C oracle where the reference exists")
    text = run_driver(REF_DRIVER)
    with open(OUT, "w", encoding="utf-8") as f:
        f.write(text)
    print(f"wrote {OUT}: {len(text.splitlines())} cases")


if __name__ == "__main__":
    main()
