// test_api.cpp -- TinyGNN's C++ API (include/tinygnn/*.hpp) on the device.
//
// Known answers from the reference's own tests (file:line per case), the
// reference's error contract, host/device coherence of Tensor views, and
// Model::forward against the layer-by-layer API.  Run by
// tests/test_cpp_api_gpu.py; exit status 0 = all checks passed.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tinygnn/graph_loader.hpp"
#include "tinygnn/layers.hpp"
#include "tinygnn/model.hpp"
#include "tinygnn/ops.hpp"
#include "tinygnn/tensor.hpp"

using namespace tinygnn;

static int g_pass = 0, g_fail = 0;

#define CHECK(cond)                                                              \
    do {                                                                         \
        if (cond) {                                                              \
            ++g_pass;                                                            \
        } else {                                                                 \
            ++g_fail;                                                            \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
        }                                                                        \
    } while (0)

#define CHECK_NEAR(a, b, tol) CHECK(std::fabs(double(a) - double(b)) <= (tol))

template <typename E>
static void check_throws(const char* what, const std::string& needle,
                         const std::function<void()>& fn, int line) {
    try {
        fn();
        ++g_fail;
        std::printf("FAIL line %d: %s did not throw\n", line, what);
    } catch (const E& e) {
        if (std::string(e.what()).find(needle) != std::string::npos) {
            ++g_pass;
        } else {
            ++g_fail;
            std::printf("FAIL line %d: %s threw '%s', expected '%s'\n", line, what, e.what(),
                        needle.c_str());
        }
    } catch (const std::exception& e) {
        ++g_fail;
        std::printf("FAIL line %d: %s threw the wrong type: %s\n", line, what, e.what());
    }
}
#define CHECK_THROWS(E, needle, stmt) check_throws<E>(#stmt, needle, [&] { stmt; }, __LINE__)

static Tensor undirected(std::size_t n, const std::vector<std::pair<int, int>>& e) {
    std::vector<std::pair<int32_t, int32_t>> both;
    for (auto& p : e) {
        both.push_back({p.first, p.second});
        both.push_back({p.second, p.first});
    }
    return GraphLoader::edge_list_to_csr(both, n);
}

static void test_tensor() {
    Tensor t = Tensor::dense(2, 3, {1, 2, 3, 4, 5, 6});
    CHECK(t.rows() == 2 && t.cols() == 3 && t.numel() == 6 && t.format() == StorageFormat::Dense);
    CHECK(t.at(1, 2) == 6.0f);
    CHECK(t.repr() == "Tensor(2x3, Dense, 24 bytes)");
    CHECK_THROWS(std::out_of_range, "out of range", t.at(2, 0));
    // tensor.cpp:46-86 validation, reference messages
    CHECK_THROWS(std::invalid_argument, "row_ptr.size() (3) must equal rows+1 (4)",
                 Tensor::sparse_csr(3, 3, {0, 1, 1}, {0}, {1.0f}));
    CHECK_THROWS(std::invalid_argument, "col_ind[1] = 5 is out of bounds for cols=3",
                 Tensor::sparse_csr(2, 3, {0, 1, 2}, {0, 5}, {1.0f, 1.0f}));
    CHECK_THROWS(std::invalid_argument, "row_ptr must be non-decreasing",
                 Tensor::sparse_csr(2, 3, {0, 2, 1}, {0}, {1.0f}));
    // coherence: device results read back, host edits reach the device
    Tensor x = Tensor::dense(1, 4, {-1, 2, -3, 4});
    relu_inplace(x);
    CHECK(!x.host_valid());
    CHECK(x.data()[0] == 0.0f && x.data()[1] == 2.0f && x.data()[3] == 4.0f);
    x.data()[0] = -7.0f;  // host edit after a device op
    relu_inplace(x);
    CHECK(x.at(0, 0) == 0.0f);
    Tensor y = x;  // value semantics: an independent copy
    y.data()[1] = 9.0f;
    CHECK(x.at(0, 1) == 2.0f && y.at(0, 1) == 9.0f);
}

static void test_ops() {
    // test_spmm.cpp:198-222 style: A = [[1,0,2],[0,3,0],[4,0,5]]
    Tensor A = Tensor::sparse_csr(3, 3, {0, 2, 3, 5}, {0, 2, 1, 0, 2}, {1, 2, 3, 4, 5});
    Tensor B = Tensor::dense(3, 2, {1, 2, 3, 4, 5, 6});
    Tensor C = spmm(A, B);
    const std::vector<float> want = {11, 14, 9, 12, 29, 38};
    for (int i = 0; i < 6; ++i) CHECK(C.data()[i] == want[i]);
    CHECK_THROWS(std::invalid_argument, "dimension mismatch", spmm(A, Tensor::dense(2, 2)));
    CHECK_THROWS(std::invalid_argument, "SparseCSR", spmm(B, B));
    Tensor M = matmul(Tensor::dense(2, 2, {1, 2, 3, 4}), Tensor::dense(2, 1, {5, 6}));
    CHECK(M.data()[0] == 17.0f && M.data()[1] == 39.0f);
    CHECK_THROWS(std::invalid_argument, "dimension mismatch",
                 matmul(Tensor::dense(2, 3), Tensor::dense(2, 3)));
    Tensor X = Tensor::dense(2, 2, {1, 2, 3, 4});
    add_bias(X, Tensor::dense(1, 2, {10, 20}));
    CHECK(X.at(1, 1) == 24.0f);
    CHECK_THROWS(std::invalid_argument, "bias must be shape (1×2)",
                 add_bias(X, Tensor::dense(1, 3)));
    Tensor Z = Tensor::dense(3, 0);
    CHECK_THROWS(std::invalid_argument, "0 columns", softmax_inplace(Z));
    Tensor S = Tensor::dense(1, 3, {1, 2, 3});
    softmax_inplace(S);
    CHECK_NEAR(S.data()[0] + S.data()[1] + S.data()[2], 1.0, 1e-6);
    Tensor L = Tensor::dense(1, 2, {0, 0});
    log_softmax_inplace(L);
    CHECK_NEAR(L.at(0, 0), std::log(0.5), 1e-6);
}

static void test_graph() {
    // graph_loader semantics: row = src, sorted, duplicates kept
    Tensor g = GraphLoader::edge_list_to_csr({{2, 1}, {0, 3}, {2, 0}, {1, 3}, {2, 1}}, 4);
    CHECK((g.row_ptr() == std::vector<int32_t>{0, 1, 2, 5, 5}));
    CHECK((g.col_ind() == std::vector<int32_t>{3, 3, 0, 1, 1}));
    CHECK_THROWS(std::invalid_argument, "edge[1].dst = 9 out of range [0, 4)",
                 GraphLoader::edge_list_to_csr({{0, 1}, {1, 9}}, 4));
    // test_gcn.cpp:288-327: path graph
    Tensor An = gcn_norm(undirected(3, {{0, 1}, {1, 2}}));
    CHECK(An.nnz() == 7);
    const double s6 = 1.0 / std::sqrt(6.0);
    const std::vector<double> w = {0.5, s6, s6, 1.0 / 3, s6, s6, 0.5};
    for (int i = 0; i < 7; ++i) CHECK_NEAR(An.data()[i], w[i], 1e-6);
    Tensor sl = add_self_loops(undirected(3, {{0, 1}, {1, 2}}));
    CHECK(sl.nnz() == 7 && sl.data()[0] == 1.0f);
    CHECK_THROWS(std::invalid_argument, "square",
                 add_self_loops(Tensor::sparse_csr(2, 3, {0, 0, 0}, {}, {})));
    Tensor es = edge_softmax(Tensor::sparse_csr(2, 2, {0, 2, 2}, {0, 1}, {0.0f, 0.0f}));
    CHECK_NEAR(es.data()[0], 0.5, 1e-6);
}

static void test_layers() {
    Tensor A = undirected(3, {{0, 1}, {1, 2}});
    Tensor H = Tensor::dense(3, 2, {1, 0, 0, 1, 1, 1});
    // test_gcn.cpp:514-543
    GCNLayer gcn(2, 2, true, Activation::ReLU);
    gcn.set_weight(Tensor::dense(2, 2, {1, 0.5f, 0.5f, 1}));
    gcn.set_bias(Tensor::dense(1, 2, {0.1f, -0.1f}));
    Tensor o = gcn.forward(gcn_norm(A), H);
    const float g[] = {0.804124f, 0.558248f, 1.287287f, 1.049829f, 1.054124f, 1.058248f};
    for (int i = 0; i < 6; ++i) CHECK_NEAR(o.data()[i], g[i], 1e-4);
    CHECK_THROWS(std::invalid_argument, "GCNLayer::set_weight: expected shape (2×2), got (3×2).",
                 gcn.set_weight(Tensor::dense(3, 2)));
    CHECK_THROWS(std::invalid_argument, "H has 3 columns but layer expects in_features=2",
                 gcn.forward(gcn_norm(A), Tensor::dense(3, 3)));
    // test_graphsage.cpp:362-383 (mean) and :509-526 (max)
    SAGELayer sage(2, 2, SAGELayer::Aggregator::Mean, true, Activation::ReLU);
    sage.set_weight_neigh(Tensor::dense(2, 2, {1, 0.5f, 0.5f, 1}));
    sage.set_weight_self(Tensor::dense(2, 2, {0.5f, 0, 0, 0.5f}));
    sage.set_bias(Tensor::dense(1, 2, {0.1f, -0.1f}));
    Tensor s = sage.forward(A, H);
    const float sm[] = {1.1f, 0.9f, 1.35f, 1.4f, 1.1f, 1.4f};
    for (int i = 0; i < 6; ++i) CHECK_NEAR(s.data()[i], sm[i], 1e-4);
    SAGELayer smax(2, 2, SAGELayer::Aggregator::Max, false, Activation::None);
    smax.set_weight_neigh(Tensor::dense(2, 2, {1, 0, 0, 1}));
    smax.set_weight_self(Tensor::dense(2, 2, {1, 0, 0, 1}));
    Tensor mx = smax.forward(A, H);
    const float mw[] = {1, 1, 1, 2, 1, 2};
    for (int i = 0; i < 6; ++i) CHECK_NEAR(mx.data()[i], mw[i], 1e-5);
    CHECK_THROWS(std::invalid_argument, "use_bias=false", smax.set_bias(Tensor::dense(1, 2)));
    Tensor agg = sage_max_aggregate(A, H);
    CHECK(agg.at(1, 0) == 1.0f && agg.at(1, 1) == 1.0f && agg.at(0, 1) == 1.0f);
    // test_gat.cpp:332-358
    GATLayer gat(2, 2, 0.2f, false, Activation::None);
    gat.set_weight(Tensor::dense(2, 2, {1, 0, 0, 1}));
    gat.set_attn_left(Tensor::dense(1, 2, {1, 0}));
    gat.set_attn_right(Tensor::dense(1, 2, {0, 1}));
    Tensor ga = gat.forward(add_self_loops(undirected(2, {{0, 1}})), Tensor::dense(2, 2, {1, 0, 0, 1}));
    const double e1 = std::exp(1.0), e2 = std::exp(2.0);
    CHECK_NEAR(ga.at(0, 0), e1 / (e1 + e2), 1e-5);
    CHECK_NEAR(ga.at(0, 1), e2 / (e1 + e2), 1e-5);
    CHECK_NEAR(ga.at(1, 0), 1 / (1 + e1), 1e-5);
    // test_gat.cpp:457-491: isolated node, bias and ReLU
    GATLayer gb(2, 2, 0.2f, true, Activation::ReLU);
    gb.set_weight(Tensor::dense(2, 2, {1, 0, 0, 1}));
    gb.set_bias(Tensor::dense(1, 2, {0.5f, -3.0f}));
    Tensor iso = add_self_loops(Tensor::sparse_csr(1, 1, {0, 0}, {}, {}));
    Tensor gbo = gb.forward(iso, Tensor::dense(1, 2, {1, 2}));
    CHECK_NEAR(gbo.at(0, 0), 1.5, 1e-5);
    CHECK_NEAR(gbo.at(0, 1), 0.0, 1e-5);
}

static void test_model() {
    Model empty;
    CHECK_THROWS(std::runtime_error, "Model::forward: no layers configured.",
                 empty.forward(Tensor::sparse_csr(1, 1, {0, 0}, {}, {}), Tensor::dense(1, 1)));
    // 2-layer GCN through Model == layer by layer (model.cpp:359-439)
    std::vector<std::pair<int32_t, int32_t>> e;
    for (int i = 0; i < 40; ++i) {
        e.push_back({i, (i * 7 + 3) % 40});
        e.push_back({(i * 7 + 3) % 40, i});
        e.push_back({i, (i + 1) % 40});
    }
    Tensor A = GraphLoader::edge_list_to_csr(e, 40);
    std::vector<float> xv(40 * 5), w0(5 * 8), w1(8 * 3), b0(8), b1(3);
    for (size_t i = 0; i < xv.size(); ++i) xv[i] = std::sin(0.37f * i);
    for (size_t i = 0; i < w0.size(); ++i) w0[i] = std::cos(0.11f * i) * 0.5f;
    for (size_t i = 0; i < w1.size(); ++i) w1[i] = std::sin(0.23f * i) * 0.5f;
    for (size_t i = 0; i < b0.size(); ++i) b0[i] = 0.01f * i;
    for (size_t i = 0; i < b1.size(); ++i) b1[i] = -0.02f * i;
    Tensor X = Tensor::dense(40, 5, xv);
    Model m;
    CHECK(m.add_gcn_layer(5, 8) == 0);
    CHECK(m.add_gcn_layer(8, 3, true, Activation::None) == 1);
    CHECK(m.num_layers() == 2);
    WeightFile wf;
    wf.tensors["layer0.weight"] = Tensor::dense(5, 8, w0);
    wf.tensors["layer0.bias"] = Tensor::dense(1, 8, b0);
    wf.tensors["layer1.weight"] = Tensor::dense(8, 3, w1);
    WeightFile missing = wf;
    CHECK_THROWS(std::runtime_error, "missing tensor 'layer1.bias'", m.load_weights(missing));
    wf.tensors["layer1.bias"] = Tensor::dense(1, 3, b1);
    m.load_weights(wf);
    Tensor out = m.forward(A, X);
    GCNLayer l0(5, 8), l1(8, 3, true, Activation::None);
    l0.set_weight(Tensor::dense(5, 8, w0));
    l0.set_bias(Tensor::dense(1, 8, b0));
    l1.set_weight(Tensor::dense(8, 3, w1));
    l1.set_bias(Tensor::dense(1, 3, b1));
    Tensor An = gcn_norm(A);
    Tensor ref = l1.forward(An, l0.forward(An, X));
    CHECK(out.data() == ref.data());
    // the cached path: same result again; an in-place edit of the adjacency
    // values must be seen (the derived adjacency is recomputed)
    Tensor out2 = m.forward(A, X);
    CHECK(out2.data() == out.data());
    A.data()[0] = 5.0f;
    Tensor out3 = m.forward(A, X);
    Tensor ref3 = l1.forward(gcn_norm(A), l0.forward(gcn_norm(A), X));
    CHECK(out3.data() == ref3.data());
    CHECK(out3.data() != out.data());
    // layers added after a forward, on the same adjacency at the same
    // version: the derived state must follow the new layer list (A's row
    // plan for SAGE, A + I for GAT); the reference's forward keeps no state,
    // so this order is legal there (model.cpp:359-439)
    CHECK(m.add_sage_layer(3, 4) == 2);
    CHECK(m.add_gat_layer(4, 2) == 3);
    std::vector<float> wn(12), ws(12), b2(4), w3(8);
    for (size_t i = 0; i < wn.size(); ++i) wn[i] = std::sin(0.3f * i + 0.1f);
    for (size_t i = 0; i < ws.size(); ++i) ws[i] = std::cos(0.2f * i) * 0.7f;
    for (size_t i = 0; i < b2.size(); ++i) b2[i] = 0.05f * i - 0.1f;
    for (size_t i = 0; i < w3.size(); ++i) w3[i] = std::sin(0.5f * i) * 0.6f;
    wf.tensors["layer2.weight_neigh"] = Tensor::dense(3, 4, wn);
    wf.tensors["layer2.weight_self"] = Tensor::dense(3, 4, ws);
    wf.tensors["layer2.bias"] = Tensor::dense(1, 4, b2);
    wf.tensors["layer3.head0.weight"] = Tensor::dense(4, 2, w3);
    wf.tensors["layer3.head0.attn_left"] = Tensor::dense(1, 2, {0.3f, -0.4f});
    wf.tensors["layer3.head0.attn_right"] = Tensor::dense(1, 2, {0.2f, 0.1f});
    wf.tensors["layer3.head0.bias"] = Tensor::dense(1, 2, {0.01f, -0.02f});
    m.load_weights(wf);
    Tensor out4 = m.forward(A, X);
    SAGELayer l2(3, 4);
    l2.set_weight_neigh(Tensor::dense(3, 4, wn));
    l2.set_weight_self(Tensor::dense(3, 4, ws));
    l2.set_bias(Tensor::dense(1, 4, b2));
    GATLayer l3(4, 2);
    l3.set_weight(Tensor::dense(4, 2, w3));
    l3.set_attn_left(Tensor::dense(1, 2, {0.3f, -0.4f}));
    l3.set_attn_right(Tensor::dense(1, 2, {0.2f, 0.1f}));
    l3.set_bias(Tensor::dense(1, 2, {0.01f, -0.02f}));
    Tensor ref4 = l3.forward(add_self_loops(A), l2.forward(A, ref3));
    CHECK(out4.rows() == 40 && out4.cols() == 2);
    for (size_t i = 0; i < ref4.data().size(); ++i)
        CHECK_NEAR(out4.data()[i], ref4.data()[i], 1e-5 + 1e-4 * std::fabs(ref4.data()[i]));
    Tensor out5 = m.forward(A, X);  // cached again with the four layers
    CHECK(out5.data() == out4.data());
    // multi-head GAT concat + ELU, then a 1-head GAT
    Model gm;
    gm.add_gat_layer(5, 4, 2, true, 0.2f, true, Activation::None, Model::InterActivation::ELU);
    gm.add_gat_layer(8, 3, 1);
    WeightFile gw;
    for (int h = 0; h < 2; ++h) {
        const std::string p = "layer0.head" + std::to_string(h);
        gw.tensors[p + ".weight"] = Tensor::dense(5, 4, std::vector<float>(w0.begin(), w0.begin() + 20));
        gw.tensors[p + ".attn_left"] = Tensor::dense(1, 4, {0.1f, -0.2f, 0.3f, 0.05f * h});
        gw.tensors[p + ".attn_right"] = Tensor::dense(1, 4, {-0.1f, 0.2f, 0.1f, 0.0f});
        gw.tensors[p + ".bias"] = Tensor::dense(1, 4);
    }
    gw.tensors["layer1.head0.weight"] = Tensor::dense(8, 3, w1);
    gw.tensors["layer1.head0.attn_left"] = Tensor::dense(1, 3, {0.2f, 0.1f, 0.0f});
    gw.tensors["layer1.head0.attn_right"] = Tensor::dense(1, 3, {0.0f, 0.3f, -0.1f});
    gw.tensors["layer1.head0.bias"] = Tensor::dense(1, 3, b1);
    gm.load_weights(gw);
    Tensor go = gm.forward(A, X);
    CHECK(go.rows() == 40 && go.cols() == 3);
    bool finite = true;
    for (float v : go.data()) finite = finite && std::isfinite(v);
    CHECK(finite);
}

// ---- ingestion (reference tests/test_graph_loader.cpp, model.cpp:49-185) ----
static std::string write_file(const std::string& name, const std::string& content) {
    const std::string path = "/tmp/tinygnn_api_test_" + name;
    std::ofstream f(path, std::ios::binary);
    f << content;
    return path;
}

template <typename T>
static void put(std::string& s, T v) {
    s.append(reinterpret_cast<const char*>(&v), sizeof v);
}

static void test_ingest() {
    // test_graph_loader.cpp:151-172
    const std::string ep = write_file("edges.csv",
                                      "src,dst\n0,1\n0,2\n1,0\n1,3\n2,0\n2,3\n2,4\n3,1\n3,2\n4,2\n");
    auto edges = GraphLoader::parse_edges(ep);
    CHECK(edges.size() == 10u);
    CHECK(edges[0] == std::make_pair(0, 1) && edges[6] == std::make_pair(2, 4) &&
          edges[9] == std::make_pair(4, 2));
    // :186-193 CRLF and spaces
    auto crlf = GraphLoader::parse_edges(write_file("crlf.csv", "src,dst\r\n0, 1\r\n1 ,0\r\n"));
    CHECK(crlf.size() == 2u && crlf[0] == std::make_pair(0, 1) && crlf[1] == std::make_pair(1, 0));
    // :228-249
    const std::string fp = write_file("feat.csv",
                                      "node_id,feat_0,feat_1,feat_2\n0,1.0,0.0,0.5\n1,0.0,1.0,0.0\n"
                                      "2,0.5,0.5,1.0\n3,0.0,0.0,1.0\n4,1.0,1.0,0.0\n");
    Tensor x = GraphLoader::parse_features(fp);
    CHECK(x.format() == StorageFormat::Dense && x.rows() == 5 && x.cols() == 3);
    CHECK(x.at(0, 0) == 1.0f && x.at(0, 2) == 0.5f && x.at(2, 1) == 0.5f && x.at(4, 2) == 0.0f);
    // :268-283 sparse ids
    Tensor sp = GraphLoader::parse_features(write_file("sparse.csv", "node_id,f0\n0,10.0\n5,50.0\n"));
    CHECK(sp.rows() == 6 && sp.at(1, 0) == 0.0f && sp.at(5, 0) == 50.0f);
    // :508-548 full pipeline
    GraphData gd = GraphLoader::load(ep, fp);
    CHECK(gd.num_nodes == 5 && gd.num_edges == 10 && gd.num_features == 3);
    CHECK(gd.adjacency.format() == StorageFormat::SparseCSR && gd.adjacency.nnz() == 10);
    CHECK(gd.node_features.at(2, 2) == 1.0f);
    const std::vector<int32_t> rp = {0, 2, 4, 7, 9, 10};  // :330-372
    CHECK(gd.adjacency.row_ptr() == rp);
    // :644-663 edges beyond the feature rows
    GraphData g2 = GraphLoader::load(write_file("e2.csv", "0,5\n5,0\n"),
                                     write_file("f2.csv", "node_id,f0\n0,1.0\n1,2.0\n"));
    CHECK(g2.num_nodes == 6 && g2.node_features.rows() == 6 && g2.node_features.at(1, 0) == 2.0f &&
          g2.node_features.at(5, 0) == 0.0f);
    // :1546-1640 errors
    CHECK_THROWS(std::runtime_error, "GraphLoader: cannot open file 'nonexistent_edges_file.csv'",
                 GraphLoader::parse_edges("nonexistent_edges_file.csv"));
    CHECK_THROWS(std::runtime_error, "file is empty", GraphLoader::parse_edges(write_file("empty.csv", "")));
    CHECK_THROWS(std::runtime_error, "malformed line 1: '0 1'",
                 GraphLoader::parse_edges(write_file("bad1.csv", "0 1\n")));
    CHECK_THROWS(std::runtime_error, "invalid integer on line 1: '0,abc'",
                 GraphLoader::parse_edges(write_file("bad2.csv", "0,abc\n")));
    CHECK_THROWS(std::runtime_error, "negative node ID on line 1: src=-1, dst=2",
                 GraphLoader::parse_edges(write_file("bad3.csv", "-1,2\n")));
    CHECK_THROWS(std::runtime_error, "inconsistent feature count on line 2: expected 2 but got 1",
                 GraphLoader::parse_features(write_file("bad4.csv", "0,1.0,2.0\n1,3.0\n")));
    CHECK_THROWS(std::runtime_error, "no data rows",
                 GraphLoader::parse_features(write_file("bad5.csv", "node_id,f0,f1\n")));
    CHECK(GraphLoader::parse_edges(write_file("hdr.csv", "src,dst\n")).empty());

    // TGNN weight file (model.hpp:22-33) and Model::load_weights(path)
    std::string wb = "TGNN";
    put<uint32_t>(wb, 1);
    put<float>(wb, 0.75f);
    put<uint32_t>(wb, 2);
    const std::vector<std::pair<std::string, std::vector<float>>> ts = {
        {"layer0.weight", {0.5f, -1.0f, 2.0f, 0.25f, 1.5f, -0.5f}}, {"layer0.bias", {0.1f, -0.2f}}};
    const uint32_t shapes[2][2] = {{3, 2}, {1, 2}};
    for (int i = 0; i < 2; ++i) {
        put<uint32_t>(wb, static_cast<uint32_t>(ts[i].first.size()));
        wb += ts[i].first;
        put<uint32_t>(wb, shapes[i][0]);
        put<uint32_t>(wb, shapes[i][1]);
        wb.append(reinterpret_cast<const char*>(ts[i].second.data()), ts[i].second.size() * 4);
    }
    const std::string wp = write_file("w.bin", wb);
    WeightFile wf = load_weight_file(wp);
    CHECK(wf.test_accuracy == 0.75f && wf.tensors.size() == 2);
    CHECK(wf.tensors.at("layer0.weight").rows() == 3 && wf.tensors.at("layer0.weight").at(2, 1) == -0.5f);
    Model m1, m2;
    m1.add_gcn_layer(3, 2, true, Activation::None);
    m2.add_gcn_layer(3, 2, true, Activation::None);
    m1.load_weights(wf);
    m2.load_weights(wp);
    Tensor A = undirected(4, {{0, 1}, {1, 2}, {2, 3}});
    Tensor X = Tensor::dense(4, 3, {1, 0, 2, 0, 1, 1, 3, 1, 0, 1, 1, 1});
    CHECK(m1.forward(A, X).data() == m2.forward(A, X).data());
    CHECK_THROWS(std::runtime_error, "load_weight_file: invalid magic in",
                 load_weight_file(write_file("badw.bin", "XXXX" + wb.substr(4))));
    CHECK_THROWS(std::runtime_error, "load_weight_file: unexpected end of file or read error.",
                 load_weight_file(write_file("truncw.bin", wb.substr(0, wb.size() - 2))));

    // Cora binary export (model.cpp:49-129)
    std::string cb;
    const uint32_t N = 5, F = 2, Cc = 3, E = 6;
    put(cb, N);
    put(cb, F);
    put(cb, Cc);
    put(cb, E);
    for (uint32_t i = 0; i < N * F; ++i) put<float>(cb, float(i) * 0.5f);
    for (uint32_t i = 0; i < N; ++i) put<int32_t>(cb, int32_t(i % Cc));
    for (int m = 0; m < 3; ++m)
        for (uint32_t i = 0; i < N; ++i) cb.push_back(char((i + m) % 2));
    const int32_t src[E] = {0, 4, 1, 0, 3, 0}, dst[E] = {3, 2, 1, 1, 0, 2};
    for (int32_t v : src) put(cb, v);
    for (int32_t v : dst) put(cb, v);
    CoraData cd = load_cora_binary(write_file("cora.bin", cb));
    CHECK(cd.num_nodes == N && cd.num_features == F && cd.num_classes == Cc && cd.num_edges == E);
    CHECK(cd.features.at(4, 1) == 4.5f && cd.labels[4] == 1 && cd.val_mask[0] == 1);
    const std::vector<int32_t> crp = {0, 3, 4, 4, 5, 6}, cci = {1, 2, 3, 1, 0, 2};
    CHECK(cd.adjacency.row_ptr() == crp && cd.adjacency.col_ind() == cci);
    CHECK_THROWS(std::runtime_error, "load_cora_binary: cannot open", load_cora_binary("/nonexistent.bin"));
}

int main() {
    const std::pair<const char*, void (*)()> suites[] = {
        {"tensor", test_tensor}, {"ops", test_ops}, {"graph", test_graph},
        {"layers", test_layers}, {"model", test_model},
        {"ingest", test_ingest}};
    for (auto& s : suites) {
        try {
            s.second();
        } catch (const std::exception& e) {
            ++g_fail;
            std::printf("FAIL suite %s threw: %s\n", s.first, e.what());
        }
        std::printf("suite %s done (%d passed, %d failed so far)\n", s.first, g_pass, g_fail);
        std::fflush(stdout);
    }
    std::printf("%d passed, %d failed\n", g_pass, g_fail);
    return g_fail == 0 ? 0 : 1;
}
