"""Pins the CPU oracle (oracle/tg_oracle.c) before it is trusted as the checker.

Four independent kinds of check, chosen so that a plausible mistake in the
restatement (a dropped term, a swapped operand, a wrong order of rounding)
fails at least one of them:

1. the reference's own known-answer tests (expected values copied from the
   reference's tests, file:line cited per test);
2. mathematics: closed forms, invariants and brute force in float64
   (dense adjacency, fp64 products, uniform-attention == mean);
3. the committed golden fixtures written by the REAL reference compiled from
   its sources (tests/golden/make_golden.py) -- bit-for-bit;
4. where oracle/_ref/libtgref.so is present, random cases against the real
   reference -- bit-for-bit.
"""
import hashlib
import os
import sys

import numpy as np
import pytest

import oracle
from helpers import bits, random_csr

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
from golden_inputs import cora_inputs, ops_inputs  # noqa: E402

from tinygnn_amd import synth  # noqa: E402


def csr_from_dense(d):
    d = np.asarray(d, np.float32)
    rp = [0]
    ci, v = [], []
    for row in d:
        nz = np.nonzero(row)[0]
        ci += list(nz)
        v += list(row[nz])
        rp.append(len(ci))
    return oracle.CSR(d.shape[0], d.shape[1], np.array(rp, np.int32), np.array(ci, np.int32),
                      np.array(v, np.float32))


def undirected(n, edges):
    """make_undirected_csr of the reference tests (test_gcn.cpp helper)."""
    src = [a for a, b in edges] + [b for a, b in edges]
    dst = [b for a, b in edges] + [a for a, b in edges]
    return oracle.restate().edge_list_to_csr(np.array(src, np.int32), np.array(dst, np.int32), n)


def dense_of(a):
    d = np.zeros((a.n_rows, a.n_cols), np.float64)
    for i in range(a.n_rows):
        for nz in range(a.row_ptr[i], a.row_ptr[i + 1]):
            d[i, a.col_ind[nz]] += a.val[nz]
    return d


# --------------------------------------------------------------------------
# 1. Reference known answers
# --------------------------------------------------------------------------
def test_known_spmm_3x3(restate):
    """test_spmm.cpp:198-222 style hand case and fractional/negative weights
    (test_spmm.cpp:1029-1047)."""
    a = csr_from_dense([[1, 0, 2], [0, 3, 0], [4, 0, 5]])
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    np.testing.assert_array_equal(restate.spmm(a, b), [[11, 14], [9, 12], [29, 38]])
    a = csr_from_dense([[0.5, -1.5], [0, 0.25]])
    b = np.array([[2, -4], [1, 8]], np.float32)
    np.testing.assert_array_equal(restate.spmm(a, b), [[-0.5, -14.0], [0.25, 2.0]])


def test_known_gcn_norm_path(restate):
    """test_gcn.cpp:288-327: path graph 0-1-2."""
    a = restate.gcn_norm(undirected(3, [(0, 1), (1, 2)]))
    assert a.nnz == 7
    np.testing.assert_array_equal(a.row_ptr, [0, 2, 5, 7])
    np.testing.assert_array_equal(a.col_ind, [0, 1, 0, 1, 2, 1, 2])
    s6 = 1 / np.sqrt(6)
    np.testing.assert_allclose(a.val, [0.5, s6, s6, 1 / 3, s6, s6, 0.5], atol=1e-5)


def test_known_gcn_norm_complete_ring_star(restate):
    """test_gcn.cpp:330-363 (K3 -> 1/3), :828-858 (ring -> 1/3),
    :966-1007 (star with 9 leaves: 1/10, 1/sqrt(20), 0.5)."""
    k3 = restate.gcn_norm(undirected(3, [(0, 1), (0, 2), (1, 2)]))
    np.testing.assert_allclose(k3.val, np.full(9, 1 / 3), atol=1e-6)
    ring = restate.gcn_norm(undirected(6, [(i, (i + 1) % 6) for i in range(6)]))
    np.testing.assert_allclose(ring.val, np.full(18, 1 / 3), atol=1e-6)
    star = restate.gcn_norm(undirected(10, [(0, i) for i in range(1, 10)]))
    d = dense_of(star)
    assert abs(d[0, 0] - 0.1) < 1e-6
    np.testing.assert_allclose(d[0, 1:], 1 / np.sqrt(20), atol=1e-6)
    np.testing.assert_allclose(d[1:, 0], 1 / np.sqrt(20), atol=1e-6)
    np.testing.assert_allclose(np.diag(d)[1:], 0.5, atol=1e-6)


def test_known_gcn_forward_3node(restate):
    """test_gcn.cpp:514-543."""
    a = restate.gcn_norm(undirected(3, [(0, 1), (1, 2)]))
    h = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    out = restate.gcn_layer(a, h, np.array([[1, .5], [.5, 1]], np.float32),
                            np.array([[.1, -.1]], np.float32), act=1)
    np.testing.assert_allclose(out, [[0.804124, 0.558248], [1.287287, 1.049829],
                                     [1.054124, 1.058248]], atol=1e-4)


def test_known_sage_mean_and_max_3node(restate):
    """test_graphsage.cpp:362-383 (mean) and :509-526 (max)."""
    a = undirected(3, [(0, 1), (1, 2)])
    h = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    out = restate.sage_layer(a, h, np.array([[1, .5], [.5, 1]], np.float32),
                             np.array([[.5, 0], [0, .5]], np.float32),
                             np.array([[.1, -.1]], np.float32), act=1, agg=0)
    np.testing.assert_allclose(out, [[1.1, 0.9], [1.35, 1.4], [1.1, 1.4]], atol=1e-4)
    eye = np.eye(2, dtype=np.float32)
    out = restate.sage_layer(a, h, eye, eye, None, act=0, agg=1)
    np.testing.assert_allclose(out, [[1, 1], [1, 2], [1, 2]], atol=1e-5)


def test_known_gat_2node_and_bias(restate):
    """test_gat.cpp:332-358 (2-node closed form; a_l is the centre vector)
    and :457-491 (isolated node: bias, ReLU)."""
    a = restate.add_self_loops(undirected(2, [(0, 1)]))
    h = np.eye(2, dtype=np.float32)
    out = restate.gat_layer(a, h, np.eye(2, dtype=np.float32), np.array([1, 0], np.float32),
                            np.array([0, 1], np.float32), None, 0.2, 0)
    e1, e2 = np.exp(1.0), np.exp(2.0)
    np.testing.assert_allclose(out[0], [e1 / (e1 + e2), e2 / (e1 + e2)], atol=1e-5)
    np.testing.assert_allclose(out[1], [1 / (1 + e1), e1 / (1 + e1)], atol=1e-5)
    iso = restate.add_self_loops(oracle.CSR(1, 1, np.zeros(2, np.int32),
                                            np.zeros(0, np.int32), np.zeros(0, np.float32)))
    h1 = np.array([[1, 2]], np.float32)
    z = np.zeros(2, np.float32)
    out = restate.gat_layer(iso, h1, np.eye(2, dtype=np.float32), z, z,
                            np.array([0.5, -0.5], np.float32), 0.2, 0)
    np.testing.assert_allclose(out, [[1.5, 1.5]], atol=1e-5)
    out = restate.gat_layer(iso, h1, np.eye(2, dtype=np.float32), z, z,
                            np.array([0.5, -3.0], np.float32), 0.2, 1)
    np.testing.assert_allclose(out, [[1.5, 0.0]], atol=1e-5)


def test_known_edge_list_to_csr(restate):
    """test_graph_loader.cpp:330-500 semantics: row = src, sorted columns,
    duplicates kept, values 1, out-of-range endpoints rejected."""
    a = restate.edge_list_to_csr(np.array([2, 0, 2, 1, 2], np.int32),
                                 np.array([1, 3, 0, 3, 1], np.int32), 4)
    np.testing.assert_array_equal(a.row_ptr, [0, 1, 2, 5, 5])
    np.testing.assert_array_equal(a.col_ind, [3, 3, 0, 1, 1])
    np.testing.assert_array_equal(a.val, np.ones(5))
    with pytest.raises(oracle.OracleError, match="out of range"):
        restate.edge_list_to_csr(np.array([0, 4], np.int32), np.array([1, 1], np.int32), 4)
    with pytest.raises(oracle.OracleError, match="out of range"):
        restate.edge_list_to_csr(np.array([0], np.int32), np.array([-1], np.int32), 4)


# --------------------------------------------------------------------------
# 2. Mathematics: brute force, invariants, special cases
# --------------------------------------------------------------------------
def test_math_spmm_matches_dense_product(restate):
    """spmm == dense matmul of the densified A (test_spmm.cpp:652-724), checked
    in fp64 with the sequential-summation error bound."""
    rng = np.random.default_rng(1)
    a = random_csr(rng, 120, 90, avg_deg=9, max_deg=80, empty_frac=0.1)
    b = rng.standard_normal((90, 33)).astype(np.float32)
    got = restate.spmm(a, b).astype(np.float64)
    d = dense_of(a)
    exact = d @ b.astype(np.float64)
    bound = (np.diff(a.row_ptr)[:, None] + 1) * 2.0 ** -24 * (np.abs(d) @ np.abs(b)) + 1e-30
    assert (np.abs(got - exact) <= bound).all()


def test_checker_spmm_rows_f64(restate):
    """The full-size tests' float64 checker against per-term brute force on
    selected rows (duplicate columns with values of either sign included,
    so sum|terms| differs from |A| @ |B|), and the float32 spmm against the
    bound it yields."""
    rng = np.random.default_rng(5)
    a = random_csr(rng, 80, 30, avg_deg=14, max_deg=60, empty_frac=0.1)
    b = rng.standard_normal((30, 9)).astype(np.float32)
    rows = np.array([79, 0, 3, 41, 41, 17], np.int32)
    exact, absum = restate.spmm_rows_f64(a, b, rows)
    for k, i in enumerate(rows):
        s, e = a.row_ptr[i], a.row_ptr[i + 1]
        terms = a.val[s:e].astype(np.float64)[:, None] * b[a.col_ind[s:e]].astype(np.float64)
        np.testing.assert_allclose(exact[k], terms.sum(0), rtol=0, atol=1e-12)
        np.testing.assert_allclose(absum[k], np.abs(terms).sum(0), rtol=0, atol=1e-12)
    got = restate.spmm(a, b)[rows].astype(np.float64)
    bound = (np.diff(a.row_ptr)[rows][:, None] + 1) * 2.0 ** -24 * absum + 1e-30
    assert (np.abs(got - exact) <= bound).all()


def test_math_matmul_fp64(restate):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((31, 57)).astype(np.float32)
    b = rng.standard_normal((57, 19)).astype(np.float32)
    got = restate.matmul(a, b).astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = 58 * 2.0 ** -24 * (np.abs(a) @ np.abs(b))
    assert (np.abs(got - exact) <= bound).all()
    # a transposed operand would fail: A^T-like shape mixup is caught by shape
    assert got.shape == (31, 19)


def test_math_self_loops_and_norm_dense(restate):
    """add_self_loops == A + I as dense matrices (every diagonal duplicate gets
    +1, missing diagonals are inserted in sorted position); gcn_norm ==
    D^-1/2 (A+I) D^-1/2 with row-sum degrees."""
    rng = np.random.default_rng(3)
    a = random_csr(rng, 60, 60, avg_deg=4, empty_frac=0.2)
    # plant diagonals, including duplicates
    extra_r = np.array([5, 5, 9, 20], np.int32)
    src = np.concatenate([np.repeat(np.arange(60), np.diff(a.row_ptr)), extra_r])
    dst = np.concatenate([a.col_ind, extra_r])
    a = restate.edge_list_to_csr(src.astype(np.int32), dst.astype(np.int32), 60)
    a.val[:] = rng.random(a.nnz).astype(np.float32) + 0.5
    sl = restate.add_self_loops(a)
    ndiag = sum(1 for i in range(60) if i not in a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]])
    assert sl.nnz == a.nnz + ndiag
    for i in range(60):
        r = sl.col_ind[sl.row_ptr[i]:sl.row_ptr[i + 1]]
        assert (np.diff(r) >= 0).all() and (r == i).any()
    d = dense_of(a)
    diag_dups = np.array([(a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]] == i).sum() for i in range(60)])
    want = d + np.diag(np.where(diag_dups > 0, diag_dups, 1))
    np.testing.assert_allclose(dense_of(sl), want, rtol=1e-6)
    gn, deg, dis = restate.gcn_norm(a, with_degrees=True)
    np.testing.assert_allclose(deg, dense_of(sl).sum(1), rtol=1e-6)
    np.testing.assert_array_equal(bits(dis), bits(np.float32(1) / np.sqrt(deg)))
    dd = 1 / np.sqrt(dense_of(sl).sum(1))
    np.testing.assert_allclose(dense_of(gn), dd[:, None] * dense_of(sl) * dd[None, :],
                               rtol=1e-5)


def test_math_softmax_invariants(restate):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((40, 23)) * 5).astype(np.float32)
    s = restate.activation("softmax", x)
    np.testing.assert_allclose(s.sum(1), 1, atol=1e-5)
    ls = restate.activation("log_softmax", x)
    np.testing.assert_allclose(np.exp(ls.astype(np.float64)).sum(1), 1, atol=1e-5)
    exact = x - (x.max(1, keepdims=True) +
                 np.log(np.exp(x.astype(np.float64) - x.max(1, keepdims=True)).sum(1,
                                                                              keepdims=True)))
    np.testing.assert_allclose(ls, exact, atol=2e-5)
    a = random_csr(rng, 50, 50, avg_deg=5, empty_frac=0.2)
    es = restate.edge_softmax(a)
    for i in range(50):
        seg = es.val[a.row_ptr[i]:a.row_ptr[i + 1]]
        if seg.size:
            assert abs(seg.sum() - 1) < 1e-5


def test_math_activation_closed_forms(restate):
    x = np.array([[-3, -1, -0.5, 0, 0.5, 1, 3]], np.float32)
    np.testing.assert_array_equal(restate.activation("relu", x), np.maximum(x, 0))
    np.testing.assert_allclose(restate.activation("leaky_relu", x, 0.2),
                               np.where(x >= 0, x, 0.2 * x), rtol=1e-7)
    np.testing.assert_allclose(restate.activation("elu", x, 1.0),
                               np.where(x < 0, np.expm1(x.astype(np.float64)), x), atol=1e-6)
    np.testing.assert_allclose(restate.activation("sigmoid", x),
                               1 / (1 + np.exp(-x.astype(np.float64))), atol=1e-6)


def test_math_gat_uniform_attention_is_mean(restate):
    """a_l = a_r = 0 makes every score equal, so GAT == mean of the neighbour
    rows of H*W (test_gat.cpp:370-394)."""
    rng = np.random.default_rng(5)
    a = restate.add_self_loops(random_csr(rng, 70, 70, avg_deg=6, empty_frac=0.1))
    h = rng.standard_normal((70, 9)).astype(np.float32)
    w = rng.standard_normal((9, 6)).astype(np.float32)
    z = np.zeros(6, np.float32)
    out = restate.gat_layer(a, h, w, z, z, None, 0.2, 0).astype(np.float64)
    wh = h.astype(np.float64) @ w.astype(np.float64)
    for i in range(70):
        cols = a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]]
        np.testing.assert_allclose(out[i], wh[cols].mean(0), atol=1e-4)


def test_math_gat_roles_brute_force(restate):
    """Scores e_ij = LeakyReLU(a_l.Wh_i + a_r.Wh_j), softmax over row i's
    neighbours j, out_i = sum alpha_ij Wh_j, all in fp64.  Swapping a_l and
    a_r, or the slope sign, fails this check."""
    rng = np.random.default_rng(6)
    a = restate.add_self_loops(random_csr(rng, 40, 40, avg_deg=5))
    h = rng.standard_normal((40, 7)).astype(np.float32)
    w = rng.standard_normal((7, 5)).astype(np.float32)
    al = rng.standard_normal(5).astype(np.float32)
    ar = rng.standard_normal(5).astype(np.float32)
    out = restate.gat_layer(a, h, w, al, ar, None, 0.2, 0).astype(np.float64)
    wh = h.astype(np.float64) @ w.astype(np.float64)
    s, d = wh @ al, wh @ ar
    for i in range(40):
        cols = a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]]
        e = s[i] + d[cols]
        e = np.where(e >= 0, e, 0.2 * e)
        p = np.exp(e - e.max())
        p /= p.sum()
        np.testing.assert_allclose(out[i], p @ wh[cols], atol=1e-4)


def test_math_sage_mean_brute_force(restate):
    rng = np.random.default_rng(7)
    a = random_csr(rng, 50, 50, avg_deg=4, empty_frac=0.2)
    h = rng.standard_normal((50, 12)).astype(np.float32)
    wn = rng.standard_normal((12, 10)).astype(np.float32)
    ws = rng.standard_normal((12, 10)).astype(np.float32)
    b = rng.standard_normal(10).astype(np.float32)
    out = restate.sage_layer(a, h, wn, ws, b, act=0, agg=0).astype(np.float64)
    for i in range(50):
        cols = a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]]
        agg = h[cols].astype(np.float64).mean(0) if cols.size else np.zeros(12)
        np.testing.assert_allclose(out[i], agg @ wn + h[i].astype(np.float64) @ ws + b,
                                   atol=1e-4)


# --------------------------------------------------------------------------
# 3. Golden fixtures written by the compiled reference
# --------------------------------------------------------------------------
def _sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


@pytest.fixture(scope="module")
def cora():
    g = np.load(os.path.join(GOLDEN, "cora_synth.npz"))
    inp = cora_inputs()
    sha = _sha(inp["src"], inp["dst"], inp["x"],
               *[inp["weights"][k][1][n] for k in sorted(inp["weights"])
                 for n in sorted(inp["weights"][k][1])])
    assert str(g["input_sha"]) == sha, "synthetic generator drifted from the fixture"
    return g, inp


def test_golden_cora_graph(restate, cora):
    g, inp = cora
    a = restate.edge_list_to_csr(inp["src"], inp["dst"], synth.CORA_NODES)
    assert a.nnz == 10858
    np.testing.assert_array_equal(a.row_ptr, g["row_ptr"])
    np.testing.assert_array_equal(a.col_ind, g["col_ind"])
    sl = restate.add_self_loops(a)
    assert sl.nnz == 13566
    np.testing.assert_array_equal(sl.row_ptr, g["sl_row_ptr"])
    np.testing.assert_array_equal(sl.col_ind, g["sl_col_ind"])
    np.testing.assert_array_equal(bits(sl.val), bits(g["sl_val"]))
    np.testing.assert_array_equal(bits(restate.gcn_norm(a).val), bits(g["norm_val"]))


@pytest.mark.parametrize("model", ["gcn", "sage", "gat"])
def test_golden_cora_forward(restate, cora, model):
    g, inp = cora
    a = restate.edge_list_to_csr(inp["src"], inp["dst"], synth.CORA_NODES)
    spec, w = inp["weights"][model]
    out = restate.model_forward(spec, w, a, inp["x"])
    np.testing.assert_array_equal(bits(out), bits(g[f"{model}_forward"]))


def test_golden_ops(restate):
    g = np.load(os.path.join(GOLDEN, "ops_small.npz"))
    inp = ops_inputs()
    assert str(g["input_sha"]) == _sha(*[inp[k] for k in sorted(inp)
                                         if isinstance(inp[k], np.ndarray)])
    a = oracle.CSR(int(inp["a_n"]), int(inp["a_k"]), inp["a_rp"], inp["a_ci"], inp["a_v"])
    np.testing.assert_array_equal(bits(restate.spmm(a, inp["b"])), bits(g["spmm"]))
    np.testing.assert_array_equal(bits(restate.matmul(inp["ma"], inp["mb"])), bits(g["matmul"]))
    for kind in ("relu", "sigmoid", "tanh", "gelu", "softmax", "log_softmax"):
        np.testing.assert_array_equal(bits(restate.activation(kind, inp["x"])),
                                      bits(g[f"act_{kind}"]), err_msg=kind)
    np.testing.assert_array_equal(bits(restate.activation("leaky_relu", inp["x"], 0.2)),
                                  bits(g["act_leaky_relu"]))
    np.testing.assert_array_equal(bits(restate.activation("elu", inp["x"], 1.0)),
                                  bits(g["act_elu"]))
    np.testing.assert_array_equal(bits(restate.add_bias(inp["x"], inp["bias_x"])),
                                  bits(g["add_bias"]))
    sq = oracle.CSR(int(inp["s_n"]), int(inp["s_n"]), inp["s_rp"], inp["s_ci"], inp["s_v"])
    np.testing.assert_array_equal(bits(restate.edge_softmax(sq).val), bits(g["edge_softmax"]))
    sl = restate.add_self_loops(sq)
    np.testing.assert_array_equal(sl.row_ptr, g["sl_row_ptr"])
    np.testing.assert_array_equal(sl.col_ind, g["sl_col_ind"])
    np.testing.assert_array_equal(bits(sl.val), bits(g["sl_val"]))
    np.testing.assert_array_equal(bits(restate.gcn_norm(sq).val), bits(g["norm_val"]))
    n = sq.n_rows
    for f in inp["gat_widths"]:
        rng = np.random.default_rng(int(f))
        h = rng.standard_normal((n, 5)).astype(np.float32)
        w = rng.standard_normal((5, int(f))).astype(np.float32)
        al = rng.standard_normal((1, int(f))).astype(np.float32)
        ar = rng.standard_normal((1, int(f))).astype(np.float32)
        b = rng.standard_normal((1, int(f))).astype(np.float32)
        got = restate.gat_layer(sl, h, w, al, ar, b, 0.2, 1)
        np.testing.assert_array_equal(bits(got), bits(g[f"gat_f{f}"]), err_msg=f"F={f}")
    h = inp["lh"]
    np.testing.assert_array_equal(
        bits(restate.gcn_layer(restate.gcn_norm(sq), h, inp["lw"], inp["lb"], 1)),
        bits(g["gcn_layer"]))
    np.testing.assert_array_equal(
        bits(restate.sage_layer(sq, h, inp["lw"], inp["lw2"], inp["lb"], 1, 0)),
        bits(g["sage_mean"]))
    np.testing.assert_array_equal(
        bits(restate.sage_layer(sq, h, inp["lw"], inp["lw2"], inp["lb"], 0, 1)),
        bits(g["sage_max"]))
    np.testing.assert_array_equal(bits(restate.sage_max_aggregate(sq, h)),
                                  bits(g["sage_max_aggregate"]))


# --------------------------------------------------------------------------
# 4. Random cases against the compiled reference (where it is built)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reference_random_graph_ops(restate, reference, seed):
    rng = np.random.default_rng(50 + seed)
    n = 300
    src = rng.integers(0, n, size=2500).astype(np.int32)
    dst = rng.integers(0, n, size=2500).astype(np.int32)
    a = restate.edge_list_to_csr(src, dst, n)
    r = reference.edge_list_to_csr(src, dst, n)
    np.testing.assert_array_equal(a.row_ptr, r.row_ptr)
    np.testing.assert_array_equal(a.col_ind, r.col_ind)
    a.val[:] = (rng.random(a.nnz) * 2).astype(np.float32)
    for fn in ("add_self_loops", "gcn_norm", "edge_softmax"):
        x, y = getattr(restate, fn)(a), getattr(reference, fn)(a)
        np.testing.assert_array_equal(x.row_ptr, y.row_ptr, err_msg=fn)
        np.testing.assert_array_equal(x.col_ind, y.col_ind, err_msg=fn)
        np.testing.assert_array_equal(bits(x.val), bits(y.val), err_msg=fn)
    for f in (1, 7, 8, 9, 33, 64):
        b = rng.standard_normal((n, f)).astype(np.float32)
        np.testing.assert_array_equal(bits(restate.spmm(a, b)), bits(reference.spmm(a, b)))


@pytest.mark.parametrize("f_in,f_out", [(5, 3), (16, 8), (17, 9), (33, 41), (64, 64)])
def test_reference_random_layers(restate, reference, f_in, f_out):
    rng = np.random.default_rng(f_in * 100 + f_out)
    n = 150
    a = random_csr(rng, n, n, avg_deg=6, max_deg=60, empty_frac=0.1)
    h = rng.standard_normal((n, f_in)).astype(np.float32)
    w = rng.standard_normal((f_in, f_out)).astype(np.float32)
    w2 = rng.standard_normal((f_in, f_out)).astype(np.float32)
    b = rng.standard_normal(f_out).astype(np.float32)
    al = rng.standard_normal(f_out).astype(np.float32)
    ar = rng.standard_normal(f_out).astype(np.float32)
    np.testing.assert_array_equal(bits(restate.matmul(h, w)), bits(reference.matmul(h, w)))
    an = restate.gcn_norm(a)
    np.testing.assert_array_equal(bits(restate.gcn_layer(an, h, w, b, 1)),
                                  bits(reference.gcn_layer(an, h, w, b, 1)))
    for agg in (0, 1):
        np.testing.assert_array_equal(bits(restate.sage_layer(a, h, w, w2, b, 1, agg)),
                                      bits(reference.sage_layer(a, h, w, w2, b, 1, agg)))
    sl = restate.add_self_loops(a)
    np.testing.assert_array_equal(bits(restate.gat_layer(sl, h, w, al, ar, b, 0.2, 1)),
                                  bits(reference.gat_layer(sl, h, w, al, ar, b, 0.2, 1)))


def test_reference_model_heads(restate, reference):
    """Multi-head GAT concat and average, SAGE-max, post activations."""
    rng = np.random.default_rng(9)
    n = 120
    a = random_csr(rng, n, n, avg_deg=5, empty_frac=0.05)
    x = rng.standard_normal((n, 12)).astype(np.float32)
    spec = [dict(type="gat", **{"in": 12}, out=5, heads=3, concat=True, slope=0.2, act=0,
                 post=2),
            dict(type="gat", **{"in": 15}, out=4, heads=2, concat=False, slope=0.1, act=1,
                 post=1),
            dict(type="sage", **{"in": 4}, out=6, agg=1, act=1, post=0),
            dict(type="gcn", **{"in": 6}, out=3, act=0, post=0)]
    w = synth.model_weights(spec, seed=5)
    for k in w:
        if k.endswith("bias"):
            w[k] = rng.standard_normal(w[k].shape).astype(np.float32)
    got = restate.model_forward(spec, w, a, x)
    want = reference.model(spec, w).forward(a, x)
    np.testing.assert_array_equal(bits(got), bits(want))


def test_reference_error_messages(reference):
    """The messages the C-ABI must reproduce (test_spmm.cpp / test_gcn.cpp
    ASSERT_THROWS_MSG substrings)."""
    a = oracle.CSR(3, 4, np.array([0, 1, 2, 3], np.int32), np.array([0, 1, 2], np.int32),
                   np.ones(3, np.float32))
    with pytest.raises(oracle.OracleError, match="dimension mismatch"):
        reference.spmm(a, np.ones((3, 2), np.float32))
    with pytest.raises(oracle.OracleError, match="square"):
        reference.add_self_loops(a)
