"""Dense transforms and epilogues on the GPU vs the oracle.

In-order matmul (reference src/ops.cpp:70-162): bit-exact.  MFMA matmul:
within the fp32 summation bound |err| <= (k+2) 2^-24 sum|a||b| of the exact
product.  Activations without a transcendental (relu, leaky_relu, add_bias)
are bit-exact; those that call exp/log/tanh use the device math library
and are held to |got - want| <= 1e-5 + 1e-4 |want| (the north-star
tolerance); the reference calls glibc's, so bitwise equality is not
expected there.
"""
import numpy as np
import pytest

import oracle
from helpers import assert_close, bits, random_csr

pytestmark = pytest.mark.gpu


def _t(gpu, x):
    return gpu.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 3, 7), (37, 41, 16), (130, 602, 41),
                                   (64, 1433, 16), (300, 256, 41), (257, 17, 64),
                                   (100, 64, 7), (513, 33, 300), (1000, 77, 24),
                                   (2708, 1433, 64),
                                   # above 2^21 outputs: the large in-order kernels
                                   (9000, 40, 300), (70000, 33, 31), (300000, 9, 8)])
def test_matmul_inorder_bitexact(gpu, restate, m, k, n):
    import tinygnn_amd as tg
    rng = np.random.default_rng(m * 31 + k * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = tg.matmul(_t(gpu, a), _t(gpu, b), algo=tg.GEMM_INORDER).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(restate.matmul(a, b)))


@pytest.mark.parametrize("m,k,n", [(128, 16, 128), (1000, 602, 256), (777, 256, 41),
                                   (300, 33, 130), (64, 1433, 64),
                                   # thin products (n <= 64: 16-column MFMA tiles), k not a
                                   # multiple of the 32-wide chunk, m not of 64
                                   (4099, 37, 16), (1000, 256, 48), (130, 300, 33), (64, 64, 60),
                                   (65, 19, 3), (2500, 256, 41)])
def test_matmul_mfma_bound(gpu, m, k, n):
    import tinygnn_amd as tg
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = tg.matmul(_t(gpu, a), _t(gpu, b), algo=tg.GEMM_MFMA).cpu().numpy().astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = (k + 2) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b)) + 1e-30
    assert (np.abs(got - exact) <= bound).all(), float((np.abs(got - exact) / bound).max())


@pytest.mark.parametrize("n", [96, 41])
@pytest.mark.parametrize("algo", [1, 2])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_matmul_epilogue(gpu, restate, algo, epi, n):
    """Fused bias + act equals add_bias then relu/elu (ops.cpp:622, :328, :380);
    n = 41 takes the thin MFMA kernel."""
    import tinygnn_amd as tg
    rng = np.random.default_rng(10 + epi + n)
    a = rng.standard_normal((200, 70)).astype(np.float32)
    b = rng.standard_normal((70, n)).astype(np.float32)
    bias = rng.standard_normal((1, n)).astype(np.float32)
    got = tg.matmul(_t(gpu, a), _t(gpu, b), bias=_t(gpu, bias), epilogue=epi,
                    algo=algo).cpu().numpy()
    want = restate.add_bias(restate.matmul(a, b), bias)
    if epi == 1:
        want = restate.activation("relu", want)
    elif epi == 2:
        want = restate.activation("elu", want, 1.0)
    if algo == 1 and epi != 2:
        np.testing.assert_array_equal(bits(got), bits(want))
    else:
        assert_close(got, want, rtol=1e-4, atol=1e-4, what="matmul epilogue")


def test_activations(gpu, restate):
    import tinygnn_amd as tg
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((333, 41)) * 4).astype(np.float32)
    x[0, :6] = [0.0, -0.0, 1e-30, -1e-30, 80.0, -80.0]
    exact = {"relu": tg.relu_, "leaky_relu": lambda t: tg.leaky_relu_(t, 0.2)}
    for name, fn in exact.items():
        got = fn(_t(gpu, x)).cpu().numpy()
        want = restate.activation(name, x, 0.2)
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=name)
    for name, fn in {"elu": lambda t: tg.elu_(t, 1.0), "sigmoid": tg.sigmoid_,
                     "tanh": tg.tanh_, "gelu": tg.gelu_}.items():
        got = fn(_t(gpu, x)).cpu().numpy()
        assert_close(got, restate.activation(name, x, 1.0), what=name)
    for name, fn in {"softmax": tg.softmax_, "log_softmax": tg.log_softmax_}.items():
        got = fn(_t(gpu, x)).cpu().numpy()
        assert_close(got, restate.activation(name, x), what=name)
    bias = rng.standard_normal((1, 41)).astype(np.float32)
    got = tg.add_bias_(_t(gpu, x), _t(gpu, bias)).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(restate.add_bias(x, bias)))


def test_activation_errors(gpu):
    import tinygnn_amd as tg
    z = gpu.zeros((3, 0), device="cuda")
    with pytest.raises(tg.InvalidArgument, match="softmax_inplace: tensor has 0 columns"):
        tg.softmax_(z)
    with pytest.raises(tg.InvalidArgument, match="log_softmax_inplace: tensor has 0 columns"):
        tg.log_softmax_(z)
    with pytest.raises(tg.InvalidArgument, match=r"add_bias: bias must be shape \(1×4\)"):
        tg.add_bias_(gpu.zeros((2, 4), device="cuda"), gpu.zeros((1, 3), device="cuda"))


def test_edge_softmax(gpu, restate):
    import tinygnn_amd as tg
    rng = np.random.default_rng(5)
    a = random_csr(rng, 500, 500, avg_deg=9, max_deg=400, empty_frac=0.2)
    a.val[:] = (rng.standard_normal(a.nnz) * 3).astype(np.float32)
    got = tg.edge_softmax(tg.DeviceCSR.from_numpy(a.n_rows, a.n_cols, a.row_ptr, a.col_ind,
                                                  a.val)).val.cpu().numpy()
    assert_close(got, restate.edge_softmax(a).val, what="edge_softmax")
    rows = np.repeat(np.arange(500), np.diff(a.row_ptr))
    sums = np.bincount(rows, weights=got.astype(np.float64), minlength=500)
    nonempty = np.diff(a.row_ptr) > 0
    np.testing.assert_allclose(sums[nonempty], 1.0, atol=1e-5)
