"""Graph preprocessing on the GPU vs the oracle -- all bit-exact.

edge_list_to_csr (reference src/graph_loader.cpp:211-281), CSR validation
(src/tensor.cpp:46-86), add_self_loops (src/layers.cpp:71-144) and gcn_norm
(src/layers.cpp:158-208), including the degree and 1/sqrt(deg) arrays.
"""
import numpy as np
import pytest

import oracle
from helpers import bits, random_csr

pytestmark = pytest.mark.gpu


def _dev(gpu, a):
    import tinygnn_amd as tg
    return tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, a.val)


def _edges(gpu, src, dst):
    return (gpu.from_numpy(np.ascontiguousarray(src, np.int32)).cuda(),
            gpu.from_numpy(np.ascontiguousarray(dst, np.int32)).cuda())


@pytest.mark.parametrize("n,e,dmax,seed", [
    (1, 0, 1, 0), (5, 1, 1, 1), (300, 4000, 64, 2), (2000, 60000, 900, 3),
    (500, 120000, 40000, 4),     # rows > 16384: the global bitonic path
    (64, 200000, 100000, 5),     # padded length 131072: several global stages
])
def test_edge_list_to_csr_bitexact(gpu, restate, n, e, dmax, seed):
    import tinygnn_amd as tg
    from tinygnn_amd import synth
    if e == 0:
        src = dst = np.zeros(0, np.int32)
    elif n <= 5:
        rng = np.random.default_rng(seed)
        src = rng.integers(0, n, size=e).astype(np.int32)
        dst = rng.integers(0, n, size=e).astype(np.int32)
    else:
        src, dst = synth.powerlaw_edges(n, e, alpha=2.1, dmax=dmax, seed=seed)
    want = restate.edge_list_to_csr(src, dst, n)
    s, d = _edges(gpu, src, dst)
    got = tg.edge_list_to_csr(s, d, n)
    rp, ci, v = got.to_numpy()
    np.testing.assert_array_equal(rp, want.row_ptr)
    np.testing.assert_array_equal(ci, want.col_ind)
    np.testing.assert_array_equal(bits(v), bits(want.val))


def test_edge_list_to_csr_duplicates_and_self_edges(gpu, restate):
    import tinygnn_amd as tg
    rng = np.random.default_rng(9)
    src = rng.integers(0, 40, size=5000).astype(np.int32)
    dst = rng.integers(0, 40, size=5000).astype(np.int32)  # many duplicates, self edges
    want = restate.edge_list_to_csr(src, dst, 40)
    got = tg.edge_list_to_csr(*_edges(gpu, src, dst), 40)
    np.testing.assert_array_equal(got.to_numpy()[0], want.row_ptr)
    np.testing.assert_array_equal(got.to_numpy()[1], want.col_ind)


@pytest.mark.parametrize("bad", [("src", 7, 10), ("dst", 3, -1), ("src", 0, 4)])
def test_edge_list_to_csr_errors(gpu, restate, bad):
    """Message of graph_loader.cpp:227-242 for the first bad endpoint."""
    import tinygnn_amd as tg
    which, pos, value = bad
    src = np.arange(12, dtype=np.int32) % 4
    dst = (np.arange(12, dtype=np.int32) + 1) % 4
    (src if which == "src" else dst)[pos] = value
    (dst if which == "src" else src)[pos + 2] = 99  # a later bad edge must not be reported
    with pytest.raises(oracle.OracleError) as want:
        restate.edge_list_to_csr(src, dst, 4)
    with pytest.raises(tg.InvalidArgument) as got:
        tg.edge_list_to_csr(*_edges(gpu, src, dst), 4)
    assert str(got.value) == str(want.value)


def test_edge_list_to_csr_zero_nodes(gpu):
    import tinygnn_amd as tg
    s, d = _edges(gpu, np.zeros(0, np.int32), np.zeros(0, np.int32))
    a = tg.edge_list_to_csr(s, d, 0)
    assert a.row_ptr.cpu().tolist() == [0]
    s, d = _edges(gpu, np.zeros(1, np.int32), np.zeros(1, np.int32))
    with pytest.raises(tg.InvalidArgument, match="num_nodes is 0 but edges is non-empty"):
        tg.edge_list_to_csr(s, d, 0)


def test_csr_validate(gpu, reference):
    import tinygnn_amd as tg
    rp = np.array([0, 2, 3, 3, 5], np.int32)
    ci = np.array([0, 3, 1, 2, 0], np.int32)
    ok = oracle.CSR(4, 4, rp, ci, np.ones(5, np.float32))
    tg.csr_validate(_dev(gpu, ok))
    cases = [
        oracle.CSR(4, 4, rp, np.array([0, 3, 1, 4, 9], np.int32), np.ones(5, np.float32)),
        oracle.CSR(4, 4, np.array([0, 2, 1, 3, 5], np.int32), ci, np.ones(5, np.float32)),
        oracle.CSR(4, 4, np.array([0, 2, 3, 3, 4], np.int32), ci[:5], np.ones(5, np.float32)),
    ]
    for c in cases:
        with pytest.raises(oracle.OracleError) as want:
            reference.csr_raw(c.n_rows, c.n_cols, c.row_ptr, c.col_ind, c.val)
        with pytest.raises(tg.InvalidArgument) as got:
            tg.csr_validate(_dev(gpu, c))
        assert str(got.value) == str(want.value)


def _graph_with_diagonals(restate, seed, n=400, unsorted=False):
    rng = np.random.default_rng(seed)
    a = random_csr(rng, n, n, avg_deg=7, max_deg=300, empty_frac=0.15)
    rows = np.repeat(np.arange(n), np.diff(a.row_ptr))
    diag = rng.choice(n, size=n // 4, replace=False)
    dup = rng.choice(diag, size=n // 20, replace=False)
    src = np.concatenate([rows, diag, dup]).astype(np.int32)
    dst = np.concatenate([a.col_ind, diag, dup]).astype(np.int32)
    g = restate.edge_list_to_csr(src, dst, n)
    g.val[:] = (rng.random(g.nnz) * 3 - 1).astype(np.float32)
    if unsorted:
        for i in range(n):
            seg = slice(g.row_ptr[i], g.row_ptr[i + 1])
            p = rng.permutation(g.row_ptr[i + 1] - g.row_ptr[i])
            g.col_ind[seg] = g.col_ind[seg][p]
            g.val[seg] = g.val[seg][p]
    return g


@pytest.mark.parametrize("seed,unsorted", [(0, False), (1, False), (2, True)])
def test_add_self_loops_bitexact(gpu, restate, seed, unsorted):
    import tinygnn_amd as tg
    a = _graph_with_diagonals(restate, seed, unsorted=unsorted)
    want = restate.add_self_loops(a)
    got = tg.add_self_loops(_dev(gpu, a))
    rp, ci, v = got.to_numpy()
    np.testing.assert_array_equal(rp, want.row_ptr)
    np.testing.assert_array_equal(ci, want.col_ind)
    np.testing.assert_array_equal(bits(v), bits(want.val))


@pytest.mark.parametrize("seed,unsorted,weights", [(3, False, "unit"), (4, False, "real"),
                                                   (5, True, "real")])
def test_gcn_norm_bitexact(gpu, restate, seed, unsorted, weights):
    import tinygnn_amd as tg
    a = _graph_with_diagonals(restate, seed, unsorted=unsorted)
    if weights == "unit":
        a.val[:] = 1.0
    else:
        a.val[:] = np.abs(a.val) + 0.01  # positive degrees, non-integer sums
    want, wdeg, wdis = restate.gcn_norm(a, with_degrees=True)
    got, deg, dis = tg.gcn_norm(_dev(gpu, a), with_degrees=True)
    rp, ci, v = got.to_numpy()
    np.testing.assert_array_equal(rp, want.row_ptr)
    np.testing.assert_array_equal(ci, want.col_ind)
    np.testing.assert_array_equal(bits(deg.cpu().numpy()), bits(wdeg))
    np.testing.assert_array_equal(bits(dis.cpu().numpy()), bits(wdis))
    np.testing.assert_array_equal(bits(v), bits(want.val))


@pytest.mark.parametrize("weights", ["unit", "real", "big_int", "neg_int"])
def test_self_loops_long_rows(gpu, restate, weights):
    """Rows up to 9,000 entries (the workgroup-per-row kernels) with
    diagonals present and absent.  Unit and small signed integers take the
    exact parallel degree; real values and integers whose magnitudes sum past
    2^24 take the sequential one."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(17)
    n = 3000
    a = random_csr(rng, n, n, avg_deg=20, max_deg=9000)
    rows = np.repeat(np.arange(n), np.diff(a.row_ptr))
    diag = rng.choice(n, size=n // 3, replace=False)
    src = np.concatenate([rows, diag]).astype(np.int32)
    dst = np.concatenate([a.col_ind, diag]).astype(np.int32)
    g = restate.edge_list_to_csr(src, dst, n)
    if weights == "unit":
        g.val[:] = 1.0
    elif weights == "real":
        g.val[:] = (rng.random(g.nnz) * 2 + 0.01).astype(np.float32)
    elif weights == "big_int":
        g.val[:] = rng.integers(1, 20000, g.nnz).astype(np.float32)
    else:
        g.val[:] = rng.integers(-5, 6, g.nnz).astype(np.float32)
    assert np.diff(g.row_ptr).max() > 2048
    want = restate.add_self_loops(g)
    rp, ci, v = tg.add_self_loops(_dev(gpu, g)).to_numpy()
    np.testing.assert_array_equal(rp, want.row_ptr)
    np.testing.assert_array_equal(ci, want.col_ind)
    np.testing.assert_array_equal(bits(v), bits(want.val))
    want, wdeg, wdis = restate.gcn_norm(g, with_degrees=True)
    got, deg, dis = tg.gcn_norm(_dev(gpu, g), with_degrees=True)
    np.testing.assert_array_equal(bits(deg.cpu().numpy()), bits(wdeg))
    np.testing.assert_array_equal(bits(dis.cpu().numpy()), bits(wdis))
    np.testing.assert_array_equal(bits(got.val.cpu().numpy()), bits(want.val))


@pytest.mark.parametrize("in_off,out_off", [(0, 1), (1, 0), (1, 1), (0, 2), (3, 0)])
def test_self_loops_pointer_alignment(gpu, restate, in_off, out_off):
    """col_ind / val inputs and outputs starting 4-12 bytes past a 16-byte
    boundary (C-ABI callers may pass any element-aligned pointer): the
    128-bit read and aligned-granule copy paths and the entry-wise ones give
    the same bits."""
    import tinygnn_amd as tg
    torch = gpu
    rng = np.random.default_rng(23)
    n = 700
    a = random_csr(rng, n, n, avg_deg=12, max_deg=3000, empty_frac=0.1)
    rows = np.repeat(np.arange(n), np.diff(a.row_ptr))
    diag = rng.choice(n, size=n // 3, replace=False)
    g = restate.edge_list_to_csr(np.concatenate([rows, diag]).astype(np.int32),
                                 np.concatenate([a.col_ind, diag]).astype(np.int32), n)
    g.val[:] = (rng.random(g.nnz) * 2 + 0.01).astype(np.float32)
    assert np.diff(g.row_ptr).max() > 2048  # the workgroup-per-row kernels too

    def placed(x, off):  # x's values in a device buffer, starting off elements in
        buf = torch.zeros(x.size + off + 4, dtype=torch.from_numpy(x[:1]).dtype).cuda()
        buf[off:off + x.size] = torch.from_numpy(x).cuda()
        return buf, buf.data_ptr() + off * x.itemsize

    rp = torch.from_numpy(g.row_ptr).cuda()
    ci_buf, ci_p = placed(g.col_ind, in_off)
    v_buf, v_p = placed(g.val, in_off)
    cap = g.nnz + n
    for norm in (False, True):
        want = restate.gcn_norm(g) if norm else restate.add_self_loops(g)
        rp_o = torch.empty(n + 1, dtype=torch.int32).cuda()
        co_buf, co_p = placed(np.zeros(cap, np.int32), out_off)
        vo_buf, vo_p = placed(np.zeros(cap, np.float32), out_off)
        if norm:
            st = tg.lib.tg_gcn_norm(n, g.nnz, rp.data_ptr(), ci_p, v_p, rp_o.data_ptr(), co_p,
                                    vo_p, None, None, None, 0, None)
        else:
            st = tg.lib.tg_add_self_loops(n, g.nnz, rp.data_ptr(), ci_p, v_p, rp_o.data_ptr(),
                                          co_p, vo_p, None, 0, None)
        tg.lib.check(st)
        torch.cuda.synchronize()
        nnz = want.row_ptr[-1]
        np.testing.assert_array_equal(rp_o.cpu().numpy(), want.row_ptr)
        ci_o = co_buf.cpu().numpy()[out_off:out_off + nnz]
        v_o = vo_buf.cpu().numpy()[out_off:out_off + nnz]
        np.testing.assert_array_equal(ci_o, want.col_ind)
        np.testing.assert_array_equal(bits(v_o), bits(want.val))
        # nothing written outside the outputs
        assert not co_buf.cpu().numpy()[:out_off].any()
        assert not co_buf.cpu().numpy()[out_off + nnz:].any()


def test_gcn_norm_degree_sweep(gpu, restate):
    """1/sqrt(deg) correctly rounded for every integer degree 1..4096 (star-like
    rows of unit weights): the device sqrt and divide must round exactly as
    the host's."""
    import tinygnn_amd as tg
    n = 4097
    rows = np.arange(1, n)
    k = rows % 4096
    src = np.repeat(rows, k)
    start = np.repeat(np.cumsum(k) - k, k)
    dst = (np.arange(src.size) - start + src + 1) % n
    a = restate.edge_list_to_csr(src.astype(np.int32), dst.astype(np.int32), n)
    want, wdeg, wdis = restate.gcn_norm(a, with_degrees=True)
    got, deg, dis = tg.gcn_norm(_dev(gpu, a), with_degrees=True)
    np.testing.assert_array_equal(bits(dis.cpu().numpy()), bits(wdis))
    np.testing.assert_array_equal(bits(got.val.cpu().numpy()), bits(want.val))


def test_self_loops_known_answers(gpu):
    """test_gcn.cpp:288-327 path graph through the GPU path."""
    import tinygnn_amd as tg
    s, d = _edges(gpu, [0, 1, 1, 2], [1, 0, 2, 1])
    a = tg.edge_list_to_csr(s, d, 3)
    nrm = tg.gcn_norm(a)
    s6 = 1 / np.sqrt(6)
    np.testing.assert_array_equal(nrm.row_ptr.cpu().numpy(), [0, 2, 5, 7])
    np.testing.assert_allclose(nrm.val.cpu().numpy(), [0.5, s6, s6, 1 / 3, s6, s6, 0.5],
                               atol=1e-6)


def test_square_required(gpu):
    import tinygnn_amd as tg
    a = oracle.CSR(3, 4, np.array([0, 1, 1, 2], np.int32), np.array([1, 3], np.int32),
                   np.ones(2, np.float32))
    with pytest.raises(tg.InvalidArgument, match="square"):
        tg.add_self_loops(_dev(gpu, a))
