"""CSR SpMM on the GPU vs the oracle (reference src/ops.cpp:198-297).

Bar, default plans (TG_PRECISION_EXACT): every row, rows longer than the
plan's chunk included, is bit-identical to the reference's fma chain.

Bar, TG_PRECISION_FAST plans: rows of at most one chunk (<= chunk_nnz
nonzeros) are bit-identical; rows split into chunks (a regrouped sum of
per-chunk partials) are held to the fp32 summation error bound
n 2^-24 sum|terms| around the float64 product, the bound the reference's own
sequential sum obeys.  (The two sums can differ by more than
1e-5 + 1e-4 |want| where a long row cancels; the exact plans are the
reference-order path.)
"""
import numpy as np
import pytest

from helpers import bits, random_csr

pytestmark = pytest.mark.gpu


def _run(gpu, a, b, chunk=0, plan=True, precision=None):
    import tinygnn_amd as tg
    da = tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, a.val)
    db = gpu.from_numpy(b).cuda()
    p = tg.SpmmPlan(da.row_ptr, a.n_rows, a.nnz, b.shape[1], chunk) if plan else None
    if p is not None and precision is not None:
        p.set_precision(precision)
    if p is None and precision is not None:
        out = tg.spmm(da, db, precision=precision)
    else:
        out = tg.spmm(da, db, plan=p)
    gpu.cuda.synchronize()
    info = p.info() if p else None
    return out.cpu().numpy(), info


@pytest.mark.parametrize("f", [1, 2, 3, 7, 8, 16, 32, 41, 64, 100, 128, 256, 512, 602])
def test_spmm_widths_bitexact(gpu, restate, f):
    rng = np.random.default_rng(100 + f)
    a = random_csr(rng, 700, 500, avg_deg=12, max_deg=300, empty_frac=0.05)
    b = rng.standard_normal((500, f)).astype(np.float32)
    want = restate.spmm(a, b)
    got, info = _run(gpu, a, b, chunk=4096)
    assert info["n_split_rows"] == 0
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("chunk", [1, 7, 64, 256])
@pytest.mark.parametrize("f", [2, 3, 4, 41, 128, 512])
def test_spmm_split_rows_exact(gpu, restate, f, chunk):
    """Default plans: rows longer than the chunk run one workgroup each
    (gathers spread over the workgroup, the chain walked in order), so every
    row is bit-identical.  Widths cover 1-, 2- and 4-float gathers and the
    32-, 64- and 128-column tiles of that kernel (f = 512: four tiles)."""
    rng = np.random.default_rng(7 * f + chunk + 1)
    a = random_csr(rng, 400, 300, avg_deg=20, max_deg=2000, empty_frac=0.1)
    b = rng.standard_normal((300, f)).astype(np.float32)
    want = restate.spmm(a, b)
    got, info = _run(gpu, a, b, chunk=chunk)
    deg = np.diff(a.row_ptr)
    assert info["n_split_rows"] == int((deg > chunk).sum())
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("f", [1, 32, 41, 128, 300])
def test_spmm_long_rows_exact(gpu, restate, f):
    """Rows of 1,025 to 30,000 nonzeros (many LDS batches, odd and even
    batch counts, a partial last batch) under the default 1,024-entry chunk,
    against the reference's chain; empty and short rows around them."""
    import oracle
    rng = np.random.default_rng(900 + f)
    n_cols = 4000
    deg = np.concatenate([rng.integers(1025, 30001, 12), [1025, 1088, 2048, 8192 + 1],
                          rng.integers(0, 50, 200)]).astype(np.int64)
    rng.shuffle(deg)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = np.concatenate([np.sort(rng.integers(0, n_cols, d)) for d in deg]).astype(np.int32)
    val = (1.0 - rng.random(int(rp[-1]))).astype(np.float32)
    a = oracle.CSR(len(deg), n_cols, rp, ci, val)
    b = rng.standard_normal((n_cols, f)).astype(np.float32)
    got, info = _run(gpu, a, b)
    assert info["n_split_rows"] == int((deg > 1024).sum())
    np.testing.assert_array_equal(bits(got), bits(restate.spmm(a, b)))


@pytest.mark.parametrize("chunk", [1, 7, 64, 256])
@pytest.mark.parametrize("f", [4, 41, 128, 512])
def test_spmm_split_rows(gpu, restate, f, chunk):
    """TG_PRECISION_FAST plans: split rows summed from per-chunk partials."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(7 * f + chunk)
    a = random_csr(rng, 400, 300, avg_deg=20, max_deg=2000, empty_frac=0.1)
    b = rng.standard_normal((300, f)).astype(np.float32)
    want = restate.spmm(a, b)
    got, info = _run(gpu, a, b, chunk=chunk, precision=tg.PRECISION_FAST)
    deg = np.diff(a.row_ptr)
    single = deg <= chunk
    np.testing.assert_array_equal(bits(got[single]), bits(want[single]))
    assert info["n_split_rows"] == int((deg > chunk).sum())
    # Split rows add per-chunk partials: a regrouped sum.  Both it and the
    # reference's sequential sum obey the classic bound
    # |fl(sum) - sum| <= n * 2^-24 * sum|terms| (n = roundings per element).
    exact, absum = _exact_spmm(a, b)
    n_round = (deg + np.ceil(deg / chunk) + 1)[:, None]
    bound = n_round * 2.0 ** -24 * absum * 1.01 + 1e-30
    for name, x in (("gpu", got), ("reference", want)):
        err = np.abs(x.astype(np.float64) - exact)
        assert (err <= bound).all(), (name, float((err / bound).max()))


def _exact_spmm(a, b):
    """fp64 product and sum of |terms| (brute force over the nonzeros)."""
    exact = np.zeros((a.n_rows, b.shape[1]))
    absum = np.zeros_like(exact)
    rows = np.repeat(np.arange(a.n_rows), np.diff(a.row_ptr))
    terms = a.val.astype(np.float64)[:, None] * b.astype(np.float64)[a.col_ind]
    np.add.at(exact, rows, terms)
    np.add.at(absum, rows, np.abs(terms))
    return exact, absum


@pytest.mark.parametrize("f,pad", [(41, 3), (41, 7), (7, 1), (3, 1), (130, 2), (257, 3)])
@pytest.mark.parametrize("chunk", [4096, 16])
def test_spmm_padded_rows(gpu, restate, f, pad, chunk):
    """B with a padded leading dimension (ld = f + pad, a multiple of 4):
    128-bit gathers read into the row padding (filled with NaN here, which
    must never reach the output), stores stay within the f columns of a
    row-major output whose rows are not 16-byte aligned."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(f * 10 + pad + chunk)
    a = random_csr(rng, 500, 300, avg_deg=10, max_deg=400, empty_frac=0.1)
    b = rng.standard_normal((300, f)).astype(np.float32)
    bp = np.full((300, f + pad), np.nan, np.float32)
    bp[:, :f] = b
    da = tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, a.val)
    dbp = gpu.from_numpy(bp).cuda()
    want = restate.spmm(a, b)
    deg = np.diff(a.row_ptr)
    single = deg <= chunk
    for precision in (tg.PRECISION_EXACT, tg.PRECISION_FAST):
        p = tg.SpmmPlan(da.row_ptr, a.n_rows, a.nnz, f, chunk, precision=precision)
        got = tg.spmm(da, dbp[:, :f], plan=p).cpu().numpy()
        assert np.isfinite(got).all()
        if precision == tg.PRECISION_EXACT:
            np.testing.assert_array_equal(bits(got), bits(want))
        else:
            np.testing.assert_array_equal(bits(got[single]), bits(want[single]))
            np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_spmm_one_shot_and_empty(gpu, restate):
    rng = np.random.default_rng(3)
    a = random_csr(rng, 300, 200, avg_deg=5, empty_frac=0.3)
    b = rng.standard_normal((200, 24)).astype(np.float32)
    got, _ = _run(gpu, a, b, plan=False)
    np.testing.assert_array_equal(bits(got), bits(restate.spmm(a, b)))
    # the one-shot form with long rows: exact by default
    a = random_csr(rng, 200, 300, avg_deg=40, max_deg=3000, empty_frac=0.1)
    b = rng.standard_normal((300, 24)).astype(np.float32)
    assert np.diff(a.row_ptr).max() > 1024
    got, _ = _run(gpu, a, b, plan=False)
    np.testing.assert_array_equal(bits(got), bits(restate.spmm(a, b)))
    import oracle
    z = oracle.CSR(5, 4, np.zeros(6, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    got, _ = _run(gpu, z, np.ones((4, 3), np.float32), plan=False)
    assert got.shape == (5, 3) and not got.any()


def test_spmm_reference_known_answers(gpu):
    """test_spmm.cpp:198-222 (3x3 with identity-like structure) and the
    fractional / negative weights case (test_spmm.cpp:1029-1047)."""
    import oracle
    # A = [[1,0,2],[0,3,0],[4,0,5]], B = [[1,2],[3,4],[5,6]]
    a = oracle.CSR(3, 3, np.array([0, 2, 3, 5], np.int32), np.array([0, 2, 1, 0, 2], np.int32),
                   np.array([1, 2, 3, 4, 5], np.float32))
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    got, _ = _run(gpu, a, b)
    np.testing.assert_allclose(got, [[11, 14], [9, 12], [29, 38]], rtol=0, atol=1e-6)
    a = oracle.CSR(2, 2, np.array([0, 2, 3], np.int32), np.array([0, 1, 1], np.int32),
                   np.array([0.5, -1.5, 0.25], np.float32))
    b = np.array([[2, -4], [1, 8]], np.float32)
    got, _ = _run(gpu, a, b)
    np.testing.assert_allclose(got, [[-0.5, -14.0], [0.25, 2.0]], rtol=0, atol=1e-6)


@pytest.mark.parametrize("f", [7, 41, 128])
@pytest.mark.parametrize("epilogue", ["none", "relu", "elu"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_spmm_epilogue_fused(gpu, restate, f, epilogue, with_bias):
    """tg_spmm_execute_epilogue (GCNLayer::forward's spmm + add_bias + act in
    one pass, layers.cpp:319-336) against the three separate calls, bit for
    bit, and against the oracle's chain: bit-exact for none / relu, within
    the tolerance for elu (device expf vs the host's)."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(40 + f)
    a = random_csr(rng, 600, 600, avg_deg=12, max_deg=3000, empty_frac=0.05)
    b = rng.standard_normal((600, f)).astype(np.float32)
    bias = rng.standard_normal(f).astype(np.float32) if with_bias else None
    da = tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, a.val)
    db = gpu.from_numpy(b).cuda()
    dbias = gpu.from_numpy(bias).cuda() if with_bias else None
    plan = tg.SpmmPlan(da.row_ptr, a.n_rows, a.nnz, f)
    code = {"none": tg.EPI_NONE, "relu": tg.EPI_RELU, "elu": tg.EPI_ELU}[epilogue]
    fused = tg.spmm_epilogue(da, db, plan, bias=dbias, epilogue=code).cpu().numpy()
    chain = tg.spmm(da, db, plan=plan)
    if with_bias:
        tg.add_bias_(chain, dbias.reshape(1, -1))
    if epilogue == "relu":
        tg.relu_(chain)
    elif epilogue == "elu":
        tg.elu_(chain)
    np.testing.assert_array_equal(bits(fused), bits(chain.cpu().numpy()))
    want = restate.spmm(a, b)
    if with_bias:
        want = want + bias[None, :]
    if epilogue == "relu":
        want = np.where(want > 0, want, np.float32(0)).astype(np.float32)
        np.testing.assert_array_equal(bits(fused), bits(want))
    elif epilogue == "none":
        np.testing.assert_array_equal(bits(fused), bits(want.astype(np.float32)))
    else:
        want = restate.activation("elu", want.astype(np.float32), 1.0)
        np.testing.assert_allclose(fused, want, rtol=1e-6, atol=1e-7)
