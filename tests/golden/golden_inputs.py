"""Seeded inputs of the golden fixtures (shared by make_golden.py and the
tests that read the fixtures)."""
from __future__ import annotations

import numpy as np

from tinygnn_amd import synth


def cora_inputs() -> dict:
    """Configs A/B/C: the Cora-synth graph, features and the three model
    stacks with their Glorot weights (zero biases)."""
    src, dst, x = synth.cora_synth()
    weights = synth.cora_models()
    return {"src": src, "dst": dst, "x": x, "weights": weights}


def ops_inputs() -> dict:
    """Small seeded operands for the per-op fixtures."""
    rng = np.random.default_rng(4242)
    out = {}
    # rectangular CSR (rows of length 0..40) for spmm
    n, k = 37, 29
    deg = rng.integers(0, 41, size=n)
    deg[[3, 17]] = 0
    rp = np.zeros(n + 1, np.int32)
    np.cumsum(deg, out=rp[1:])
    ci = np.concatenate([np.sort(rng.integers(0, k, size=d)) for d in deg]).astype(np.int32)
    out.update(a_n=np.array(n), a_k=np.array(k), a_rp=rp, a_ci=ci,
               a_v=(rng.random(int(rp[-1])) * 2 - 1).astype(np.float32),
               b=rng.standard_normal((k, 19)).astype(np.float32))
    out["ma"] = rng.standard_normal((23, 41)).astype(np.float32)
    out["mb"] = rng.standard_normal((41, 13)).astype(np.float32)
    out["x"] = (rng.standard_normal((11, 17)) * 4).astype(np.float32)
    out["bias_x"] = rng.standard_normal((1, 17)).astype(np.float32)
    # square CSR with existing diagonals, duplicate diagonals and empty rows
    sn = 24
    rows = []
    for i in range(sn):
        d = int(rng.integers(0, 7))
        cols = list(rng.integers(0, sn, size=d))
        if i % 5 == 0:
            cols.append(i)
        if i % 7 == 0:
            cols += [i, i]
        if i in (4, 13):
            cols = []
        rows.append(sorted(int(c) for c in cols))
    srp = np.zeros(sn + 1, np.int32)
    np.cumsum([len(r) for r in rows], out=srp[1:])
    out["s_n"] = np.array(sn)
    out["s_rp"] = srp
    out["s_ci"] = np.array([c for r in rows for c in r], np.int32)
    out["s_v"] = (rng.random(int(srp[-1])) * 3 - 1).astype(np.float32)
    out["gat_widths"] = np.array(list(range(1, 18)) + [41, 64, 100])
    out["lh"] = rng.standard_normal((sn, 13)).astype(np.float32)
    out["lw"] = rng.standard_normal((13, 11)).astype(np.float32)
    out["lw2"] = rng.standard_normal((13, 11)).astype(np.float32)
    out["lb"] = rng.standard_normal((1, 11)).astype(np.float32)
    return out
