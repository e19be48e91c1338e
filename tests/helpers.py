"""Test helpers: random CSR builders and comparison utilities."""
import numpy as np

import oracle


def random_csr(rng, n_rows, n_cols, avg_deg, max_deg=None, weighted=True, empty_frac=0.0,
               sorted_cols=True):
    """CSR with a heavy-tailed degree distribution (some long rows)."""
    deg = rng.geometric(1.0 / max(avg_deg, 1.0), size=n_rows) - 1
    if max_deg is not None:
        heavy = rng.choice(n_rows, size=max(1, n_rows // 200), replace=False)
        deg[heavy] = rng.integers(max_deg // 2, max_deg + 1, size=heavy.shape[0])
    if empty_frac > 0:
        deg[rng.random(n_rows) < empty_frac] = 0
    rp = np.zeros(n_rows + 1, np.int64)
    np.cumsum(deg, out=rp[1:])
    nnz = int(rp[-1])
    ci = rng.integers(0, max(n_cols, 1), size=nnz).astype(np.int32)
    if sorted_cols:
        for i in range(n_rows):
            ci[rp[i]:rp[i + 1]].sort()
    val = (rng.random(nnz).astype(np.float32) * 2 - 1) if weighted else np.ones(nnz, np.float32)
    return oracle.CSR(n_rows, n_cols, rp.astype(np.int32), ci, val.astype(np.float32))


def assert_close(got, want, rtol=1e-4, atol=1e-5, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = atol + rtol * np.abs(want.astype(np.float64))
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} elements out of tolerance; worst at "
                             f"{i}: got {got[i]!r} want {want[i]!r}")


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.int32)
