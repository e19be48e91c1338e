"""The `tinygnn` package (pybind `_tinygnn_core` over the device C++ API) on
the GPU: the known answers of the reference's tests/test_python_bindings.py
(ops, activations, graph utilities, the three layers, Model with weight
files), parity of the same calls against the compiled reference, the
module's ingestion entry points, and zero-copy torch interop."""
import os
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tinygnn_amd")


@pytest.fixture(scope="module")
def tg(gpu):
    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import tinygnn
    return tinygnn


def triangle(tg):
    return tg.Tensor.sparse_csr(3, 3, [0, 2, 4, 6], [1, 2, 0, 2, 0, 1], [1.0] * 6)


def row(tg, vals):
    return tg.Tensor.from_numpy(np.asarray(vals, np.float32).reshape(1, -1))


def test_ops(tg):
    x = tg.Tensor.from_numpy(np.array([[1, 2], [3, 4], [5, 6]], np.float32))
    np.testing.assert_array_equal(tg.matmul(tg.Tensor.from_numpy(np.eye(3, dtype=np.float32)),
                                            x).to_numpy(), x.to_numpy())
    c = tg.matmul(tg.Tensor.from_numpy(np.array([[1, 2], [3, 4]], np.float32)),
                  tg.Tensor.from_numpy(np.array([[5, 6], [7, 8]], np.float32)))
    np.testing.assert_array_equal(c.to_numpy(), [[19, 22], [43, 50]])
    eye = tg.Tensor.sparse_csr(3, 3, [0, 1, 2, 3], [0, 1, 2], [1.0] * 3)
    np.testing.assert_array_equal(tg.spmm(eye, x).to_numpy(), x.to_numpy())
    a = tg.Tensor.sparse_csr(2, 3, [0, 2, 4], [0, 1, 1, 2], [1.0] * 4)
    b = tg.Tensor.from_numpy(np.array([[1, 0], [0, 1], [2, 2]], np.float32))
    np.testing.assert_array_equal(tg.spmm(a, b).to_numpy(), [[1, 1], [2, 3]])


def test_activations(tg):
    t = row(tg, [-2, -1, 0, 1, 2])
    tg.relu_inplace(t)
    np.testing.assert_array_equal(t.to_numpy().ravel(), [0, 0, 0, 1, 2])
    t = row(tg, [-10, 0, 10])
    tg.leaky_relu_inplace(t, 0.1)
    np.testing.assert_allclose(t.to_numpy().ravel(), [-1.0, 0.0, 10.0])
    t = row(tg, [0, 1, -1])
    tg.elu_inplace(t, 1.0)
    np.testing.assert_allclose(t.to_numpy().ravel(), [0.0, 1.0, np.exp(-1) - 1], atol=1e-6)
    for fn, want in ((tg.sigmoid_inplace, 0.5), (tg.tanh_inplace, 0.0), (tg.gelu_inplace, 0.0)):
        t = row(tg, [0])
        fn(t)
        assert abs(t.to_numpy()[0, 0] - want) < 1e-6
    t = row(tg, [1, 2, 3])
    tg.softmax_inplace(t)
    s = t.to_numpy().ravel()
    assert abs(s.sum() - 1) < 1e-6 and s[2] > s[1] > s[0]
    t = row(tg, [1, 2, 3])
    tg.log_softmax_inplace(t)
    assert abs(np.exp(t.to_numpy()).sum() - 1) < 1e-6
    x = tg.Tensor.from_numpy(np.ones((3, 2), np.float32))
    tg.add_bias(x, tg.Tensor.from_numpy(np.array([[10.0, 20.0]], np.float32)))
    np.testing.assert_array_equal(x.to_numpy(), [[11, 21]] * 3)


def test_graph_utils(tg):
    a = tg.Tensor.sparse_csr(2, 2, [0, 1, 1], [1], [1.0])
    assert tg.add_self_loops(a).nnz == 3
    for t in (tg.gcn_norm(triangle(tg)), tg.edge_softmax(triangle(tg))):
        rp, v = t.row_ptr_numpy(), t.values_numpy()
        for i in range(3):
            assert abs(v[rp[i]:rp[i + 1]].sum() - 1) < 1e-6
    h = tg.Tensor.from_numpy(np.array([[1, 0], [0, 5], [3, 2]], np.float32))
    np.testing.assert_array_equal(tg.sage_max_aggregate(triangle(tg), h).to_numpy(),
                                  [[3, 5], [3, 2], [1, 5]])


def test_layers(tg):
    an = tg.gcn_norm(triangle(tg))
    g = tg.GCNLayer(2, 2, True, tg.Activation.RELU)
    g.set_weight(tg.Tensor.from_numpy(-np.eye(2, dtype=np.float32)))
    g.set_bias(tg.Tensor.from_numpy(np.zeros((1, 2), np.float32)))
    out = g.forward(an, tg.Tensor.from_numpy(np.ones((3, 2), np.float32))).to_numpy()
    assert out.shape == (3, 2) and (out >= 0).all()
    s = tg.SAGELayer(2, 2, tg.SAGELayer.Aggregator.Mean, True, tg.Activation.NONE)
    s.set_weight_neigh(tg.Tensor.from_numpy(np.eye(2, dtype=np.float32)))
    s.set_weight_self(tg.Tensor.from_numpy(np.eye(2, dtype=np.float32)))
    s.set_bias(tg.Tensor.from_numpy(np.zeros((1, 2), np.float32)))
    np.testing.assert_allclose(s.forward(triangle(tg), tg.Tensor.from_numpy(
        np.ones((3, 2), np.float32))).to_numpy(), 2.0)
    m = tg.SAGELayer(2, 2, tg.SAGELayer.Aggregator.Max, True, tg.Activation.NONE)
    m.set_weight_neigh(tg.Tensor.from_numpy(np.eye(2, dtype=np.float32)))
    m.set_weight_self(tg.Tensor.from_numpy(np.eye(2, dtype=np.float32)))
    m.set_bias(tg.Tensor.from_numpy(np.zeros((1, 2), np.float32)))
    h = tg.Tensor.from_numpy(np.array([[1, 0], [0, 3], [2, 1]], np.float32))
    np.testing.assert_array_equal(m.forward(triangle(tg), h).to_numpy()[0], [3, 3])
    rng = np.random.default_rng(1)
    a = tg.GATLayer(4, 2, 0.2, True, tg.Activation.NONE)
    a.set_weight(tg.Tensor.from_numpy(rng.standard_normal((4, 2)).astype(np.float32) * 0.1))
    a.set_attn_left(tg.Tensor.from_numpy(rng.standard_normal((1, 2)).astype(np.float32) * 0.1))
    a.set_attn_right(tg.Tensor.from_numpy(rng.standard_normal((1, 2)).astype(np.float32) * 0.1))
    a.set_bias(tg.Tensor.from_numpy(np.zeros((1, 2), np.float32)))
    out = a.forward(tg.add_self_loops(triangle(tg)),
                    tg.Tensor.from_numpy(rng.standard_normal((3, 4)).astype(np.float32)))
    assert out.to_numpy().shape == (3, 2) and np.isfinite(out.to_numpy()).all()


def test_model_weight_files(tg, tmp_path):
    import tinygnn_amd
    rng = np.random.default_rng(42)
    m = tg.Model()
    m.add_gcn_layer(4, 3, True, tg.Activation.RELU)
    m.add_gcn_layer(3, 2, True, tg.Activation.NONE)
    assert m.num_layers == 2
    w = {"layer0.weight": rng.standard_normal((4, 3)).astype(np.float32) * 0.1,
         "layer0.bias": np.zeros((1, 3), np.float32),
         "layer1.weight": rng.standard_normal((3, 2)).astype(np.float32) * 0.1,
         "layer1.bias": np.zeros((1, 2), np.float32)}
    p = str(tmp_path / "w.bin")
    tinygnn_amd.save_weight_file(p, w, 0.92)
    m.load_weights(p)
    x = tg.Tensor.from_numpy(rng.standard_normal((3, 4)).astype(np.float32))
    out = m.forward(triangle(tg), x).to_numpy()
    assert out.shape == (3, 2) and np.isfinite(out).all()
    wf = tg.load_weight_file(p)
    assert abs(wf.test_accuracy - 0.92) < 1e-6 and set(wf.tensors) == set(w)
    assert (wf.tensors["layer0.weight"].rows, wf.tensors["layer0.weight"].cols) == (4, 3)
    m2 = tg.Model()
    m2.add_gcn_layer(4, 3, True, tg.Activation.RELU)
    m2.add_gcn_layer(3, 2, True, tg.Activation.NONE)
    m2.load_weights_from_file(wf)
    np.testing.assert_array_equal(m2.forward(triangle(tg), x).to_numpy(), out)
    s = tg.Model()
    s.add_sage_layer(4, 3)
    s.add_sage_layer(3, 2, tg.SAGELayer.Aggregator.Mean, True, tg.Activation.NONE)
    with pytest.raises(RuntimeError, match="missing tensor 'layer0.weight_neigh'"):
        s.load_weights(p)


def test_parity_with_reference(tg, reference):
    """The module's results equal the compiled reference's on the same input
    (graph preprocessing and Cora-scale layers are bit-exact)."""
    from helpers import random_csr
    rng = np.random.default_rng(3)
    n = 500
    a = random_csr(rng, n, n, avg_deg=7)
    t = tg.Tensor.sparse_csr(n, n, a.row_ptr.tolist(), a.col_ind.tolist(), a.val.tolist())
    want = reference.gcn_norm(a)
    got = tg.gcn_norm(t)
    np.testing.assert_array_equal(got.row_ptr_numpy(), want.row_ptr)
    np.testing.assert_array_equal(got.col_ind_numpy(), want.col_ind)
    np.testing.assert_array_equal(got.values_numpy().view(np.int32), want.val.view(np.int32))
    b = rng.standard_normal((n, 24)).astype(np.float32)
    np.testing.assert_array_equal(tg.spmm(t, tg.Tensor.from_numpy(b)).to_numpy().view(np.int32),
                                  reference.spmm(a, b).view(np.int32))
    ei = np.stack([rng.integers(0, n, 3000), rng.integers(0, n, 3000)]).astype(np.int32)
    e = tg.Tensor.from_edge_index(ei, n)
    w = reference.edge_list_to_csr(ei[0], ei[1], n)
    np.testing.assert_array_equal(e.row_ptr_numpy(), w.row_ptr)
    np.testing.assert_array_equal(e.col_ind_numpy(), w.col_ind)


def test_from_edge_index_errors(tg):
    ei = np.array([[0, 1, 2], [1, 7, 0]], np.int32)  # destination 7 >= 3
    with pytest.raises(ValueError, match=r"col_ind\[1\] = 7 is out of bounds for cols=3"):
        tg.Tensor.from_edge_index(ei, 3)
    ei = np.array([[0, 5, 2], [1, 1, 0]], np.int32)  # source 5 >= 3
    with pytest.raises(ValueError, match=r"from_edge_index: edge\[1\].src = 5 out of range"):
        tg.Tensor.from_edge_index(ei, 3)


def test_ingestion_through_module(tg, tmp_path):
    ep, fp = str(tmp_path / "e.csv"), str(tmp_path / "f.csv")
    open(ep, "w").write("src,dst\n0,1\n0,2\n1,0\n2,4\n")
    open(fp, "w").write("node_id,a,b\n0,1.0,2.0\n3,0.5,-1\n")
    assert tg.GraphLoader.parse_edges(ep) == [(0, 1), (0, 2), (1, 0), (2, 4)]
    x = tg.GraphLoader.parse_features(fp)
    np.testing.assert_array_equal(x.to_numpy(), [[1, 2], [0, 0], [0, 0], [0.5, -1]])
    g = tg.GraphLoader.load(ep, fp)
    assert (g.num_nodes, g.num_edges, g.num_features) == (5, 4, 2)
    np.testing.assert_array_equal(g.adjacency.row_ptr_numpy(), [0, 2, 3, 4, 4, 4])
    assert g.node_features.rows == 5
    with pytest.raises(RuntimeError, match="GraphLoader: cannot open file"):
        tg.GraphLoader.parse_edges(str(tmp_path / "none.csv"))


def test_torch_interop(tg, gpu):
    torch = gpu
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = tg.Tensor.from_numpy(a)
    v = tg.to_torch(t)  # zero-copy view of the HBM buffer
    assert v.is_cuda and tuple(v.shape) == (3, 4)
    np.testing.assert_array_equal(v.cpu().numpy(), a)
    v.mul_(2.0)  # a device write through the view ...
    torch.cuda.synchronize()
    np.testing.assert_array_equal(t.to_numpy(), 2 * a)  # ... is what the tensor holds
    back = tg.from_torch(torch.ones((2, 5), device="cuda") * 3)
    np.testing.assert_array_equal(back.to_numpy(), np.full((2, 5), 3, np.float32))
    rp, ci, val = tg.to_torch(triangle(tg))
    np.testing.assert_array_equal(rp.cpu().numpy(), [0, 2, 4, 6])
    np.testing.assert_array_equal(ci.cpu().numpy(), [1, 2, 0, 2, 0, 1])
    # a tensor produced on the device, consumed by torch without a host copy
    y = tg.spmm(triangle(tg), tg.Tensor.from_numpy(a[:, :2].copy()))
    np.testing.assert_array_equal(tg.to_torch(y).cpu().numpy(),
                                  [[a[1, 0] + a[2, 0], a[1, 1] + a[2, 1]],
                                   [a[0, 0] + a[2, 0], a[0, 1] + a[2, 1]],
                                   [a[0, 0] + a[1, 0], a[0, 1] + a[1, 1]]])
