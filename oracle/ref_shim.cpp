// ref_shim.cpp -- C-ABI driver over the REAL reference library.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
// with the reference's own sources (src/{tensor,ops,layers,model,
// graph_loader}.cpp, read in place from the reference checkout) into
// oracle/_ref/libtgref.so.  Tests use it to pin the C restatement
// (tg_oracle.c) bit-for-bit, tests/golden/make_golden.py uses it to write
// the golden fixtures, and bench.py's cpu_baseline leg times its
// Model::forward on the host cores.  Nothing in the product loads it.
//
// Every entry point catches the reference's exceptions and returns
// 1 (std::invalid_argument), 2 (std::runtime_error), 3 (std::out_of_range)
// or 4 (anything else), with what() available from ref_last_error().
#include "tinygnn/graph_loader.hpp"
#include "tinygnn/layers.hpp"
#include "tinygnn/model.hpp"
#include "tinygnn/ops.hpp"
#include "tinygnn/tensor.hpp"

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

using namespace tinygnn;

namespace {

thread_local std::string g_err;

template <typename F>
int guard(F&& fn) {
    try {
        fn();
        return 0;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return 1;
    } catch (const std::out_of_range& e) {
        g_err = e.what();
        return 3;
    } catch (const std::runtime_error& e) {
        g_err = e.what();
        return 2;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 4;
    }
}

Tensor csr(int64_t rows, int64_t cols, int64_t nnz, const int32_t* rp,
           const int32_t* ci, const float* v) {
    return Tensor::sparse_csr(
        static_cast<std::size_t>(rows), static_cast<std::size_t>(cols),
        std::vector<int32_t>(rp, rp + rows + 1),
        std::vector<int32_t>(ci, ci + nnz), std::vector<float>(v, v + nnz));
}

Tensor dense(int64_t rows, int64_t cols, const float* x) {
    return Tensor::dense(static_cast<std::size_t>(rows),
                         static_cast<std::size_t>(cols),
                         std::vector<float>(x, x + rows * cols));
}

void copy_out(const Tensor& t, float* out) {
    std::memcpy(out, t.data().data(), t.data().size() * sizeof(float));
}

struct RefModel {
    Model model;
    WeightFile wf;
};

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

void ref_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int ref_get_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// Opaque reference Tensor handles, so timed calls exclude the copies and
// CSR validation that building a Tensor from raw arrays costs.
void* ref_tensor_csr(int64_t rows, int64_t cols, int64_t nnz,
                     const int32_t* rp, const int32_t* ci, const float* v) {
    Tensor* t = nullptr;
    if (guard([&] { t = new Tensor(csr(rows, cols, nnz, rp, ci, v)); })) return nullptr;
    return t;
}

void* ref_tensor_dense(int64_t rows, int64_t cols, const float* x) {
    Tensor* t = nullptr;
    if (guard([&] { t = new Tensor(dense(rows, cols, x)); })) return nullptr;
    return t;
}

void ref_tensor_free(void* t) { delete static_cast<Tensor*>(t); }

int64_t ref_tensor_rows(void* t) { return static_cast<int64_t>(static_cast<Tensor*>(t)->rows()); }
int64_t ref_tensor_cols(void* t) { return static_cast<int64_t>(static_cast<Tensor*>(t)->cols()); }
int64_t ref_tensor_nnz(void* t) { return static_cast<int64_t>(static_cast<Tensor*>(t)->nnz()); }

int ref_tensor_read(void* t, int32_t* rp, int32_t* ci, float* v) {
    const Tensor& x = *static_cast<Tensor*>(t);
    if (rp && !x.row_ptr().empty())
        std::memcpy(rp, x.row_ptr().data(), x.row_ptr().size() * sizeof(int32_t));
    if (ci && !x.col_ind().empty())
        std::memcpy(ci, x.col_ind().data(), x.col_ind().size() * sizeof(int32_t));
    if (v && !x.data().empty()) std::memcpy(v, x.data().data(), x.data().size() * sizeof(float));
    return 0;
}

// --- graph preprocessing -------------------------------------------------
void* ref_edge_list_to_csr(int64_t n_nodes, int64_t n_edges,
                           const int32_t* src, const int32_t* dst) {
    Tensor* t = nullptr;
    if (guard([&] {
            std::vector<std::pair<int32_t, int32_t>> e(static_cast<std::size_t>(n_edges));
            for (int64_t i = 0; i < n_edges; ++i) e[i] = {src[i], dst[i]};
            t = new Tensor(GraphLoader::edge_list_to_csr(e, static_cast<std::size_t>(n_nodes)));
        }))
        return nullptr;
    return t;
}

void* ref_add_self_loops(void* a) {
    Tensor* t = nullptr;
    if (guard([&] { t = new Tensor(add_self_loops(*static_cast<Tensor*>(a))); })) return nullptr;
    return t;
}

void* ref_gcn_norm(void* a) {
    Tensor* t = nullptr;
    if (guard([&] { t = new Tensor(gcn_norm(*static_cast<Tensor*>(a))); })) return nullptr;
    return t;
}

void* ref_edge_softmax(void* a) {
    Tensor* t = nullptr;
    if (guard([&] { t = new Tensor(edge_softmax(*static_cast<Tensor*>(a))); })) return nullptr;
    return t;
}

// --- ops -----------------------------------------------------------------
int ref_spmm(void* a, void* b, float* out) {
    return guard([&] { copy_out(spmm(*static_cast<Tensor*>(a), *static_cast<Tensor*>(b)), out); });
}

int ref_matmul(void* a, void* b, float* out) {
    return guard([&] { copy_out(matmul(*static_cast<Tensor*>(a), *static_cast<Tensor*>(b)), out); });
}

int ref_sage_max_aggregate(void* a, void* h, float* out) {
    return guard([&] {
        copy_out(sage_max_aggregate(*static_cast<Tensor*>(a), *static_cast<Tensor*>(h)), out);
    });
}

// kind: 0 relu, 1 leaky_relu(alpha), 2 elu(alpha), 3 sigmoid, 4 tanh,
//       5 gelu, 6 softmax, 7 log_softmax
int ref_activation(int kind, int64_t rows, int64_t cols, float* x, float alpha) {
    return guard([&] {
        Tensor t = dense(rows, cols, x);
        switch (kind) {
            case 0: relu_inplace(t); break;
            case 1: leaky_relu_inplace(t, alpha); break;
            case 2: elu_inplace(t, alpha); break;
            case 3: sigmoid_inplace(t); break;
            case 4: tanh_inplace(t); break;
            case 5: gelu_inplace(t); break;
            case 6: softmax_inplace(t); break;
            case 7: log_softmax_inplace(t); break;
            default: throw std::invalid_argument("ref_activation: bad kind");
        }
        copy_out(t, x);
    });
}

int ref_add_bias(int64_t rows, int64_t cols, float* x, int64_t b_rows,
                 int64_t b_cols, const float* b) {
    return guard([&] {
        Tensor t = dense(rows, cols, x);
        add_bias(t, dense(b_rows, b_cols, b));
        copy_out(t, x);
    });
}

// --- layers ----------------------------------------------------------------
int ref_gcn_layer(void* a, void* h, int64_t f_in, int64_t f_out, const float* w,
                  const float* b, int use_bias, int act, float* out) {
    return guard([&] {
        GCNLayer l(static_cast<std::size_t>(f_in), static_cast<std::size_t>(f_out),
                   use_bias != 0, static_cast<Activation>(act));
        l.set_weight(dense(f_in, f_out, w));
        if (use_bias) l.set_bias(dense(1, f_out, b));
        copy_out(l.forward(*static_cast<Tensor*>(a), *static_cast<Tensor*>(h)), out);
    });
}

int ref_sage_layer(void* a, void* h, int64_t f_in, int64_t f_out, int agg,
                   const float* wn, const float* ws, const float* b, int use_bias,
                   int act, float* out) {
    return guard([&] {
        SAGELayer l(static_cast<std::size_t>(f_in), static_cast<std::size_t>(f_out),
                    static_cast<SAGELayer::Aggregator>(agg), use_bias != 0,
                    static_cast<Activation>(act));
        l.set_weight_neigh(dense(f_in, f_out, wn));
        l.set_weight_self(dense(f_in, f_out, ws));
        if (use_bias) l.set_bias(dense(1, f_out, b));
        copy_out(l.forward(*static_cast<Tensor*>(a), *static_cast<Tensor*>(h)), out);
    });
}

int ref_gat_layer(void* a, void* h, int64_t f_in, int64_t f_out, const float* w,
                  const float* al, const float* ar, const float* b, float slope,
                  int use_bias, int act, float* out) {
    return guard([&] {
        GATLayer l(static_cast<std::size_t>(f_in), static_cast<std::size_t>(f_out),
                   slope, use_bias != 0, static_cast<Activation>(act));
        l.set_weight(dense(f_in, f_out, w));
        l.set_attn_left(dense(1, f_out, al));
        l.set_attn_right(dense(1, f_out, ar));
        if (use_bias) l.set_bias(dense(1, f_out, b));
        copy_out(l.forward(*static_cast<Tensor*>(a), *static_cast<Tensor*>(h)), out);
    });
}

// --- Model ---------------------------------------------------------------
void* ref_model_create(void) { return new RefModel(); }
void ref_model_free(void* m) { delete static_cast<RefModel*>(m); }

int ref_model_add_gcn(void* m, int64_t in_f, int64_t out_f, int bias, int act, int post) {
    return guard([&] {
        static_cast<RefModel*>(m)->model.add_gcn_layer(
            static_cast<std::size_t>(in_f), static_cast<std::size_t>(out_f), bias != 0,
            static_cast<Activation>(act), static_cast<Model::InterActivation>(post));
    });
}

int ref_model_add_sage(void* m, int64_t in_f, int64_t out_f, int agg, int bias, int act,
                       int post) {
    return guard([&] {
        static_cast<RefModel*>(m)->model.add_sage_layer(
            static_cast<std::size_t>(in_f), static_cast<std::size_t>(out_f),
            static_cast<SAGELayer::Aggregator>(agg), bias != 0, static_cast<Activation>(act),
            static_cast<Model::InterActivation>(post));
    });
}

int ref_model_add_gat(void* m, int64_t in_f, int64_t out_f, int64_t heads, int concat,
                      float slope, int bias, int act, int post) {
    return guard([&] {
        static_cast<RefModel*>(m)->model.add_gat_layer(
            static_cast<std::size_t>(in_f), static_cast<std::size_t>(out_f),
            static_cast<std::size_t>(heads), concat != 0, slope, bias != 0,
            static_cast<Activation>(act), static_cast<Model::InterActivation>(post));
    });
}

int ref_model_set_tensor(void* m, const char* name, int64_t rows, int64_t cols,
                         const float* x) {
    return guard([&] { static_cast<RefModel*>(m)->wf.tensors[name] = dense(rows, cols, x); });
}

int ref_model_load_weights(void* m) {
    return guard([&] {
        RefModel* r = static_cast<RefModel*>(m);
        r->model.load_weights(r->wf);
    });
}

int ref_model_forward(void* m, void* adj, void* x, int64_t* out_rows, int64_t* out_cols,
                      float* out, int64_t out_capacity) {
    return guard([&] {
        Tensor y = static_cast<RefModel*>(m)->model.forward(*static_cast<Tensor*>(adj),
                                                             *static_cast<Tensor*>(x));
        *out_rows = static_cast<int64_t>(y.rows());
        *out_cols = static_cast<int64_t>(y.cols());
        if (out && static_cast<int64_t>(y.data().size()) <= out_capacity) copy_out(y, out);
    });
}

// --- file ingestion (graph_loader.cpp:61-326, model.cpp:49-185) -----------
// Handle-returning entry points store the guard's code in *code.
struct RefEdges {
    std::vector<std::pair<int32_t, int32_t>> e;
};

void* ref_parse_edges(const char* path, int* code) {
    RefEdges* r = nullptr;
    *code = guard([&] { r = new RefEdges{GraphLoader::parse_edges(path)}; });
    return r;
}
int64_t ref_edges_count(void* h) { return static_cast<int64_t>(static_cast<RefEdges*>(h)->e.size()); }
void ref_edges_read(void* h, int32_t* src, int32_t* dst) {
    const auto& e = static_cast<RefEdges*>(h)->e;
    for (size_t i = 0; i < e.size(); ++i) {
        src[i] = e[i].first;
        dst[i] = e[i].second;
    }
}
void ref_edges_free(void* h) { delete static_cast<RefEdges*>(h); }

void* ref_parse_features(const char* path, int* code) {
    Tensor* t = nullptr;
    *code = guard([&] { t = new Tensor(GraphLoader::parse_features(path)); });
    return t;
}

void* ref_graph_load(const char* edges_path, const char* features_path, int* code) {
    GraphData* g = nullptr;
    *code = guard([&] { g = new GraphData(GraphLoader::load(edges_path, features_path)); });
    return g;
}
void* ref_graph_adjacency(void* g) { return &static_cast<GraphData*>(g)->adjacency; }
void* ref_graph_features(void* g) { return &static_cast<GraphData*>(g)->node_features; }
void ref_graph_counts(void* g, int64_t* nodes, int64_t* edges, int64_t* features) {
    const GraphData& d = *static_cast<GraphData*>(g);
    *nodes = static_cast<int64_t>(d.num_nodes);
    *edges = static_cast<int64_t>(d.num_edges);
    *features = static_cast<int64_t>(d.num_features);
}
void ref_graph_free(void* g) { delete static_cast<GraphData*>(g); }

void* ref_load_cora(const char* path, int* code) {
    CoraData* c = nullptr;
    *code = guard([&] { c = new CoraData(load_cora_binary(path)); });
    return c;
}
void ref_cora_counts(void* h, int64_t* nodes, int64_t* features, int64_t* classes,
                     int64_t* edges) {
    const CoraData& c = *static_cast<CoraData*>(h);
    *nodes = static_cast<int64_t>(c.num_nodes);
    *features = static_cast<int64_t>(c.num_features);
    *classes = static_cast<int64_t>(c.num_classes);
    *edges = static_cast<int64_t>(c.num_edges);
}
void* ref_cora_adjacency(void* h) { return &static_cast<CoraData*>(h)->adjacency; }
void* ref_cora_features(void* h) { return &static_cast<CoraData*>(h)->features; }
void ref_cora_read(void* h, int32_t* labels, uint8_t* train, uint8_t* val, uint8_t* test) {
    const CoraData& c = *static_cast<CoraData*>(h);
    std::memcpy(labels, c.labels.data(), c.labels.size() * sizeof(int32_t));
    std::memcpy(train, c.train_mask.data(), c.train_mask.size());
    std::memcpy(val, c.val_mask.data(), c.val_mask.size());
    std::memcpy(test, c.test_mask.data(), c.test_mask.size());
}
void ref_cora_free(void* h) { delete static_cast<CoraData*>(h); }

void* ref_load_weight_file(const char* path, int* code) {
    WeightFile* w = nullptr;
    *code = guard([&] { w = new WeightFile(load_weight_file(path)); });
    return w;
}
float ref_weights_accuracy(void* h) { return static_cast<WeightFile*>(h)->test_accuracy; }
// Tensor names joined by '\n' into buf (cap bytes); returns the needed size.
int64_t ref_weights_names(void* h, char* buf, int64_t cap) {
    std::string all;
    for (const auto& kv : static_cast<WeightFile*>(h)->tensors) {
        if (!all.empty()) all += '\n';
        all += kv.first;
    }
    if (buf && cap > static_cast<int64_t>(all.size())) std::memcpy(buf, all.c_str(), all.size() + 1);
    return static_cast<int64_t>(all.size()) + 1;
}
void* ref_weights_tensor(void* h, const char* name) {
    auto& t = static_cast<WeightFile*>(h)->tensors;
    auto it = t.find(name);
    return it == t.end() ? nullptr : &it->second;
}
void ref_weights_free(void* h) { delete static_cast<WeightFile*>(h); }

}  // extern "C"
