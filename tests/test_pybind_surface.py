"""The `tinygnn` package / `_tinygnn_core` module on the CPU: the reference
package's names (python/tinygnn/__init__.py), host-side tensor construction
and observers, and argument errors raised before any device work (the cases
of the reference's tests/test_python_bindings.py that touch no kernel)."""
import os
import sys

import numpy as np
import pytest

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tinygnn_amd")


@pytest.fixture(scope="module")
def tg():
    from tinygnn_amd import build
    import glob
    if not glob.glob(os.path.join(build.BUILD, "_tinygnn_core*.so")):
        pytest.skip("_tinygnn_core not built")
    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import tinygnn
    return tinygnn


# python/tinygnn/__init__.py of the reference: the re-exported names
REFERENCE_NAMES = [
    "StorageFormat", "Activation", "Tensor", "matmul", "spmm", "relu_inplace",
    "leaky_relu_inplace", "elu_inplace", "sigmoid_inplace", "tanh_inplace", "gelu_inplace",
    "softmax_inplace", "log_softmax_inplace", "add_bias", "add_self_loops", "gcn_norm",
    "edge_softmax", "sage_max_aggregate", "GCNLayer", "SAGELayer", "GATLayer", "Model", "CoraData",
    "WeightFile", "load_cora_binary", "load_weight_file", "GraphData", "GraphLoader",
]


def test_reference_names(tg):
    for name in REFERENCE_NAMES:
        assert hasattr(tg, name), name
    core = sys.modules["_tinygnn_core"]
    for name in REFERENCE_NAMES + ["set_num_threads", "get_max_threads"]:
        assert hasattr(core, name), name


def test_dense_host_side(tg):
    t = tg.Tensor.dense(3, 4)
    assert (t.rows, t.cols, t.numel) == (3, 4, 12)
    assert t.format == tg.StorageFormat.Dense
    assert all(t.at(r, c) == 0.0 for r in range(3) for c in range(4))
    assert t.memory_footprint_bytes == 48
    assert "3x4" in t.repr() and "Dense" in t.repr() and "3x4" in repr(t)
    d = tg.Tensor.dense_from_data(2, 3, [1.0, 2.0, 3.0, 4.0, 5.0, 6.0])
    assert (d.at(0, 2), d.at(1, 0)) == (3.0, 4.0)
    a = np.random.default_rng(0).standard_normal((5, 7)).astype(np.float32)
    np.testing.assert_array_equal(tg.Tensor.from_numpy(a).to_numpy(), a)
    assert tg.Tensor.from_numpy(np.array([[1.5, 2.5]])).at(0, 1) == 2.5  # float64 cast
    v = tg.Tensor.from_numpy_1d(np.array([10, 20, 30], np.float32))
    assert (v.rows, v.cols, v.at(0, 1)) == (1, 3, 20.0)


def test_csr_host_side(tg):
    t = tg.Tensor.sparse_csr(2, 2, [0, 1, 3], [0, 0, 1], [5.0, 6.0, 7.0])
    assert t.format == tg.StorageFormat.SparseCSR and t.nnz == 3
    np.testing.assert_array_equal(t.row_ptr_numpy(), [0, 1, 3])
    np.testing.assert_array_equal(t.col_ind_numpy(), [0, 0, 1])
    np.testing.assert_array_equal(t.values_numpy(), [5.0, 6.0, 7.0])
    sp = pytest.importorskip("scipy.sparse")
    m = sp.csr_matrix((np.array([1.0, 2.0, 3.0, 4.0], np.float32),
                       (np.array([0, 0, 1, 2]), np.array([0, 2, 1, 0]))), shape=(3, 3))
    s = tg.Tensor.from_scipy_csr(m)
    assert (s.rows, s.cols, s.nnz) == (3, 3, 4)
    np.testing.assert_array_equal(s.values_numpy(), [1.0, 2.0, 3.0, 4.0])
    with pytest.raises(ValueError, match="col_ind\\[1\\] = 5 is out of bounds for cols=2"):
        tg.Tensor.sparse_csr(2, 2, [0, 1, 2], [0, 5], [1.0, 1.0])


def test_errors_before_device_work(tg):
    with pytest.raises(ValueError, match="expected 2D array, got 3D"):
        tg.Tensor.from_numpy(np.ones((2, 3, 4), np.float32))
    with pytest.raises(ValueError, match="Dense"):
        tg.Tensor.sparse_csr(1, 1, [0, 1], [0], [1.0]).to_numpy()
    with pytest.raises(ValueError, match=r"expected shape \(2, E\), got \(3, 4\)"):
        tg.Tensor.from_edge_index(np.ones((3, 4), np.int32), 5)
    with pytest.raises(IndexError):
        tg.Tensor.dense(2, 2).at(2, 0)


def test_layers_and_enums(tg):
    g = tg.GCNLayer(16, 32, True, tg.Activation.RELU)
    assert (g.in_features, g.out_features, g.has_bias, g.activation) == \
        (16, 32, True, tg.Activation.RELU)
    s = tg.SAGELayer(8, 4, tg.SAGELayer.Aggregator.Max)
    assert s.aggregator == tg.SAGELayer.Aggregator.Max and s.activation == tg.Activation.RELU
    a = tg.GATLayer(16, 8, 0.2, True, tg.Activation.NONE)
    assert abs(a.negative_slope - 0.2) < 1e-7 and a.has_bias
    assert tg.StorageFormat.Dense != tg.StorageFormat.SparseCSR
    assert tg.Activation.NONE != tg.Activation.RELU
    assert tg.Model.InterActivation.ELU != tg.Model.InterActivation.RELU
