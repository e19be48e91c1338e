"""tg_spmm_noalloc, the SpMM entry point that allocates nothing, against the
entry point it varies, tg_spmm (reference spmm, src/ops.cpp:198-297), both
called through the C-ABI.

Two calls in a row, the second on a smaller input, so that the second runs
over the scratch the first left behind: each output must equal tg_spmm's
bit for bit (the same plan and kernels), and the oracle's to the SpMM bar
(rows of one plan chunk bit-identical, split rows within the float32
summation bound of the float64 product).  Outputs start as NaN, so an
element left unwritten fails.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import bits, random_csr

pytestmark = pytest.mark.gpu


def _spmm(gpu, fn, a, b):
    """One call of tg_spmm / tg_spmm_noalloc on fresh device copies."""
    from tinygnn_amd import _lib
    import tinygnn_amd as tg
    L = _lib.lib.load()
    rp = gpu.from_numpy(a.row_ptr).cuda()
    ci = gpu.from_numpy(a.col_ind).cuda()
    v = gpu.from_numpy(a.val).cuda()
    db = gpu.from_numpy(b).cuda()
    c = gpu.full((a.n_rows, b.shape[1]), float("nan"), device="cuda:0")
    rc = getattr(L, fn)(a.n_rows, a.n_cols, b.shape[1], a.nnz, rp.data_ptr(), ci.data_ptr(),
                        v.data_ptr(), db.data_ptr(), b.shape[1], c.data_ptr(), b.shape[1],
                        C.c_void_p(tg.stream_handle()))
    assert rc == 0, L.tg_last_error().decode()
    gpu.cuda.synchronize()
    return c.cpu().numpy()


def _check_oracle(restate, a, b, got):
    want = restate.spmm(a, b)
    deg = np.diff(a.row_ptr)
    single = deg <= 1024  # the plan's chunk
    np.testing.assert_array_equal(bits(got[single]), bits(want[single]))
    rows = np.flatnonzero(~single).astype(np.int32)
    if rows.size:
        exact, absum = restate.spmm_rows_f64(a, b, rows)
        k = (deg[rows] + np.ceil(deg[rows] / 1024) + 1)[:, None]
        bound = k * 2.0 ** -24 * absum * 1.01 + 1e-30
        assert (np.abs(got[rows].astype(np.float64) - exact) <= bound).all()
    return int(rows.size)


def test_spmm_noalloc_two_calls(gpu, restate):
    rng = np.random.default_rng(77)
    big = random_csr(rng, 30_000, 26_000, avg_deg=40, max_deg=6000, empty_frac=0.05)
    b_big = rng.standard_normal((26_000, 72)).astype(np.float32)
    small = random_csr(rng, 4_000, 5_000, avg_deg=9, max_deg=2500, empty_frac=0.2)
    b_small = rng.standard_normal((5_000, 24)).astype(np.float32)
    n_split = []
    for a, b in ((big, b_big), (small, b_small)):
        got = _spmm(gpu, "tg_spmm_noalloc", a, b)
        ref = _spmm(gpu, "tg_spmm", a, b)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(bits(got), bits(ref))
        n_split.append(_check_oracle(restate, a, b, got))
    assert n_split[0] > 0 and n_split[1] > 0  # both calls reduce split rows


def test_spmm_noalloc_edges(gpu, restate):
    """No nonzeros (a zero result), a single row longer than several chunks,
    and a width that is not a multiple of 4."""
    import oracle
    z = oracle.CSR(7, 5, np.zeros(8, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    got = _spmm(gpu, "tg_spmm_noalloc", z, np.ones((5, 3), np.float32))
    assert got.shape == (7, 3) and not got.any()
    rng = np.random.default_rng(5)
    n = 5000
    ci = np.sort(rng.integers(0, n, 4500)).astype(np.int32)
    rp = np.zeros(3, np.int32)
    rp[1:] = [4500, 4500]
    a = oracle.CSR(2, n, rp, ci, rng.random(4500).astype(np.float32))
    b = rng.standard_normal((n, 41)).astype(np.float32)
    got = _spmm(gpu, "tg_spmm_noalloc", a, b)
    np.testing.assert_array_equal(bits(got), bits(_spmm(gpu, "tg_spmm", a, b)))
    assert _check_oracle(restate, a, b, got) == 1
