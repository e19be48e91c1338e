"""GraphSAGE and GAT layers on the GPU vs the oracle.

SAGE (reference src/layers.cpp:538-752): the concat dataflow with the
in-order GEMM is bit-exact for rows of at most one plan chunk (mean and
max); transform-first and split rows are within |err| <= 1e-5 + 1e-4|want|.
GAT (src/layers.cpp:945-1129): scores are bit-exact; the edge pass calls
exp on the device and reduces the softmax sum across lanes, so it is held
to the same tolerance.
"""
import numpy as np
import pytest

from helpers import assert_close, bits, random_csr

pytestmark = pytest.mark.gpu


def _t(gpu, x):
    return gpu.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def _dev(a):
    import tinygnn_amd as tg
    return tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind, a.val)


def _plan(da, max_f, chunk=0):
    import tinygnn_amd as tg
    return tg.SpmmPlan(da.row_ptr, da.n_rows, da.nnz, max_f, chunk)


@pytest.mark.parametrize("agg", [0, 1])
@pytest.mark.parametrize("f_in,f_out", [(5, 3), (13, 11), (64, 7), (100, 16), (33, 64),
                                        (37, 41), (20, 130)])
def test_sage_concat_bitexact(gpu, restate, agg, f_in, f_out):
    """The reference's dataflow, bit for bit: the aggregation in nonzero
    order, then the in-order dual GEMM (one output per thread up to 32
    columns; in 64-column slabs beyond, with scalar-tail columns from
    f_out rounded down to 8 -- 40 of 41, 128 of 130 -- and k not a multiple
    of the GEMM's k-tile)."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(agg * 1000 + f_in * 10 + f_out)
    n = 400
    a = random_csr(rng, n, n, avg_deg=8, max_deg=200, empty_frac=0.1)
    h = rng.standard_normal((n, f_in)).astype(np.float32)
    wn = rng.standard_normal((f_in, f_out)).astype(np.float32)
    ws = rng.standard_normal((f_in, f_out)).astype(np.float32)
    b = rng.standard_normal((1, f_out)).astype(np.float32)
    want = restate.sage_layer(a, h, wn, ws, b, act=1, agg=agg)
    da = _dev(a)
    got = tg.sage_forward(_plan(da, max(f_in, f_out)), da, _t(gpu, h), _t(gpu, wn), _t(gpu, ws),
                          _t(gpu, b), act=1, agg=agg, dataflow=tg.SAGE_CONCAT).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("agg", [0, 1])
def test_sage_aggregate_split_rows(gpu, restate, agg):
    import tinygnn_amd as tg
    rng = np.random.default_rng(77 + agg)
    n, f = 300, 24
    a = random_csr(rng, n, n, avg_deg=15, max_deg=1500, empty_frac=0.1)
    h = rng.standard_normal((n, f)).astype(np.float32)
    da = _dev(a)
    got = tg.sage_aggregate(_plan(da, f, chunk=64), da, _t(gpu, h), agg).cpu().numpy()
    # oracle aggregate = SAGE forward with identity Wn and zero Ws, no bias/act
    eye = np.eye(f, dtype=np.float32)
    want = restate.sage_layer(a, h, eye, np.zeros_like(eye), None, act=0, agg=agg)
    if agg == 1:
        np.testing.assert_array_equal(bits(got), bits(want))  # max is order-free
    else:
        assert_close(got, want, what="mean aggregate (split rows)")


@pytest.mark.parametrize("f_in,f_out", [(602, 256), (256, 41), (96, 40)])
def test_sage_transform_first(gpu, restate, f_in, f_out):
    import tinygnn_amd as tg
    rng = np.random.default_rng(f_in + f_out)
    n = 1200
    a = random_csr(rng, n, n, avg_deg=20, max_deg=3000, empty_frac=0.05)
    h = rng.standard_normal((n, f_in)).astype(np.float32)
    s = np.float32(1.0 / np.sqrt(f_in))
    wn = (rng.standard_normal((f_in, f_out)) * s).astype(np.float32)
    ws = (rng.standard_normal((f_in, f_out)) * s).astype(np.float32)
    b = rng.standard_normal((1, f_out)).astype(np.float32)
    want = restate.sage_layer(a, h, wn, ws, b, act=1, agg=0)
    da = _dev(a)
    got = tg.sage_forward(_plan(da, 2 * f_out), da, _t(gpu, h), _t(gpu, wn), _t(gpu, ws),
                          _t(gpu, b), act=1, agg=0,
                          dataflow=tg.SAGE_TRANSFORM_FIRST).cpu().numpy()
    assert_close(got, want, what="sage transform-first")


def test_sage_concat_mfma_dual(gpu, restate):
    """Concat dataflow large enough for the MFMA GEMM (m*n*k >= 2^32): the
    dual product [AGG | H] x [Wn ; Ws] runs as two K segments of one MFMA
    kernel; within tolerance of the reference."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(21)
    n, f_in, f_out = 40000, 256, 210
    a = random_csr(rng, n, n, avg_deg=3, max_deg=50, empty_frac=0.05)
    h = rng.standard_normal((n, f_in)).astype(np.float32)
    s = np.float32(1.0 / np.sqrt(f_in))
    wn = (rng.standard_normal((f_in, f_out)) * s).astype(np.float32)
    ws = (rng.standard_normal((f_in, f_out)) * s).astype(np.float32)
    b = rng.standard_normal((1, f_out)).astype(np.float32)
    want = restate.sage_layer(a, h, wn, ws, b, act=1, agg=0)
    da = _dev(a)
    got = tg.sage_forward(_plan(da, f_in), da, _t(gpu, h), _t(gpu, wn), _t(gpu, ws), _t(gpu, b),
                          act=1, agg=0, dataflow=tg.SAGE_CONCAT).cpu().numpy()
    assert_close(got, want, what="sage concat (MFMA dual)")


@pytest.mark.parametrize("f", [1, 2, 3, 7, 8, 9, 16, 17, 41, 64, 100])
def test_gat_scores_bitexact(gpu, restate, f):
    import tinygnn_amd as tg
    rng = np.random.default_rng(f)
    n, heads = 90, 3
    wh = rng.standard_normal((n, heads * f)).astype(np.float32)
    al = rng.standard_normal((heads, f)).astype(np.float32)
    ar = rng.standard_normal((heads, f)).astype(np.float32)
    src, dst = tg.gat_scores(_t(gpu, wh), heads, f, _t(gpu, al), _t(gpu, ar))
    for h in range(heads):
        ws, wd = restate.gat_scores(wh[:, h * f:(h + 1) * f], al[h], ar[h])
        np.testing.assert_array_equal(bits(src.cpu().numpy()[:, h]), bits(ws))
        np.testing.assert_array_equal(bits(dst.cpu().numpy()[:, h]), bits(wd))


@pytest.mark.parametrize("heads,f,pitch", [(1, 4, 0), (4, 64, 0), (5, 32, 0), (16, 64, 0),
                                            (16, 12, 0), (17, 8, 0), (1, 41, 64), (1, 41, 44),
                                            (1, 41, 0), (2, 41, 96)])
def test_gat_scores_bitexact_heads(gpu, restate, heads, f, pitch):
    """The scores at more heads and nodes: workgroups of 128 (node, head)
    pairs whose nodes straddle them, the LDS-staged path up to 16 heads of
    at most 64 features (f % 4 == 0, or one head whose rows are padded to a
    multiple of 4 floats: `pitch`, 0 = unpadded), the per-thread path past
    them."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(heads * 1000 + f)
    n = 1003
    wh = rng.standard_normal((n, heads * f)).astype(np.float32)
    al = rng.standard_normal((heads, f)).astype(np.float32)
    ar = rng.standard_normal((heads, f)).astype(np.float32)
    whd = _t(gpu, wh)
    if pitch:
        padded = gpu.full((n, pitch), float("nan"), device="cuda")
        padded[:, :heads * f] = whd
        whd = padded[:, :heads * f]  # rows `pitch` floats apart, NaN in the padding
    src, dst = tg.gat_scores(whd, heads, f, _t(gpu, al), _t(gpu, ar))
    src, dst = src.cpu().numpy(), dst.cpu().numpy()
    for h in range(heads):
        ws, wd = restate.gat_scores(wh[:, h * f:(h + 1) * f], al[h], ar[h])
        np.testing.assert_array_equal(bits(src[:, h]), bits(ws), err_msg=f"head {h}")
        np.testing.assert_array_equal(bits(dst[:, h]), bits(wd), err_msg=f"head {h}")


def _gat_case(restate, rng, n, f_in, f, heads, max_deg):
    a = restate.add_self_loops(random_csr(rng, n, n, avg_deg=10, max_deg=max_deg,
                                          empty_frac=0.05))
    h = rng.standard_normal((n, f_in)).astype(np.float32)
    w = (rng.standard_normal((heads, f_in, f)) / np.sqrt(f_in)).astype(np.float32)
    al = rng.standard_normal((heads, f)).astype(np.float32)
    ar = rng.standard_normal((heads, f)).astype(np.float32)
    b = rng.standard_normal((heads, f)).astype(np.float32)
    return a, h, w, al, ar, b


@pytest.mark.parametrize("heads,f,concat,chunk", [(1, 7, True, 0), (4, 64, True, 0),
                                                  (8, 8, True, 0), (4, 64, True, 32),
                                                  (3, 41, False, 0), (2, 16, False, 16),
                                                  (1, 41, True, 8)])
def test_gat_layer(gpu, restate, heads, f, concat, chunk):
    """All heads in one fused pass vs the reference's per-head layers
    followed by concat / average (model.cpp:312-354)."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(heads * 100 + f + chunk)
    n, f_in = 700, 24
    a, h, w, al, ar, b = _gat_case(restate, rng, n, f_in, f, heads, max_deg=400)
    outs = [restate.gat_layer(a, h, w[k], al[k], ar[k], b[k], 0.2, 1) for k in range(heads)]
    if concat:
        want = np.concatenate(outs, 1)
    else:
        acc = np.zeros_like(outs[0])
        for o in outs:
            acc += o
        want = acc * np.float32(1.0 / heads)
    wall = np.concatenate(list(w), axis=1)  # [f_in x heads*f], head-major columns
    da = _dev(a)
    whd = tg.matmul(_t(gpu, h), _t(gpu, wall), algo=tg.GEMM_INORDER)
    src, dst = tg.gat_scores(whd, heads, f, _t(gpu, al), _t(gpu, ar))
    got = tg.gat_aggregate(_plan(da, heads * f, chunk), da, whd, heads, f, src, dst, 0.2,
                           _t(gpu, b.reshape(1, -1)), act=1, concat=concat).cpu().numpy()
    assert_close(got, want, what=f"gat heads={heads} f={f} concat={concat} chunk={chunk}")


def test_gat_uniform_attention_is_mean(gpu, restate):
    """a_l = a_r = 0: every row's attention is uniform, so GAT == mean of the
    neighbours' Wh (test_gat.cpp:370-394), also for split rows."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(3)
    n, f = 500, 32
    a = restate.add_self_loops(random_csr(rng, n, n, avg_deg=12, max_deg=900))
    wh = rng.standard_normal((n, f)).astype(np.float32)
    z = np.zeros((1, f), np.float32)
    da = _dev(a)
    whd = _t(gpu, wh)
    src, dst = tg.gat_scores(whd, 1, f, _t(gpu, z), _t(gpu, z))
    got = tg.gat_aggregate(_plan(da, f, 64), da, whd, 1, f, src, dst).cpu().numpy()
    for i in range(n):
        cols = a.col_ind[a.row_ptr[i]:a.row_ptr[i + 1]]
        np.testing.assert_allclose(got[i], wh[cols].astype(np.float64).mean(0), atol=2e-5)
