// throw_sites.cpp -- drives every throw statement of the reference's
// src/{tensor,ops,layers,model,graph_loader}.cpp through TinyGNN's public C++
// API and prints, per case, the exception's type and message:
//
//   <case>\t<invalid_argument|out_of_range|runtime_error|other|none>\t<what()>
//
// The same source is compiled twice: against the reference's own sources
// (oracle/Makefile, oracle/_ref/throw_sites_ref: the expected output,
// committed as tests/golden/throw_sites.tsv) and against this build's C++
// API (tinygnn_amd/_build/test_throw_sites).  tests/test_throw_sites.py
// compares the two line by line.  graph_loader.cpp:142 ("empty line") has
// no case: read_lines keeps only non-empty trimmed lines, on which the first
// getline always succeeds, so that throw cannot be reached.
// Arguments: the mode ("host": the cases
// this build answers without a GPU; "all") and a scratch directory, which
// must be given as the same relative path in both runs (file names appear
// in the messages).  Each case names the throw site it reaches (file:line).
#include <cstdint>
#include <cstdio>
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

namespace {

struct Case {
    const char* name;
    bool device;  // this build needs a GPU to reach the check
    std::function<void()> fn;
};

void run(const Case& c) {
    std::string kind = "none", msg;
    try {
        c.fn();
    } catch (const std::invalid_argument& e) {
        kind = "invalid_argument";
        msg = e.what();
    } catch (const std::out_of_range& e) {
        kind = "out_of_range";
        msg = e.what();
    } catch (const std::runtime_error& e) {
        kind = "runtime_error";
        msg = e.what();
    } catch (const std::exception& e) {
        kind = "other";
        msg = e.what();
    }
    std::printf("%s\t%s\t%s\n", c.name, kind.c_str(), msg.c_str());
    std::fflush(stdout);
}

Tensor dn(std::size_t r, std::size_t c) { return Tensor::dense(r, c); }

// 3 x 3 CSR: one entry per row (the diagonal)
Tensor csr3() { return Tensor::sparse_csr(3, 3, {0, 1, 2, 3}, {0, 1, 2}, {1.f, 1.f, 1.f}); }
// 2 x 3 CSR (not square)
Tensor csr23() { return Tensor::sparse_csr(2, 3, {0, 1, 2}, {0, 2}, {1.f, 1.f}); }

void write_file(const std::string& path, const std::string& bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(bytes.data(), static_cast<std::streamsize>(bytes.size()));
}

std::string u32(uint32_t v) {
    std::string s(4, '\0');
    for (int i = 0; i < 4; ++i) s[i] = static_cast<char>((v >> (8 * i)) & 0xFF);
    return s;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "all";
    const std::string dir = argc > 2 ? argv[2] : ".";
    const std::string P = dir + "/";

    // files for the model.cpp / graph_loader.cpp cases
    write_file(P + "short.cora", "\x01\x02");
    write_file(P + "short.tgnn", "TGNN" + u32(1));
    write_file(P + "magic.tgnn", "TGNX" + u32(1) + u32(0));
    write_file(P + "version.tgnn", "TGNN" + u32(7) + u32(0));
    write_file(P + "empty.csv", "  \n\n");
    write_file(P + "nocomma.csv", "src,dst\n0,1\n2 3\n");
    write_file(P + "badint.csv", "0,1\n1,x\n");
    write_file(P + "negid.csv", "0,1\n-2,1\n");
    write_file(P + "header_only.csv", "node_id,f0,f1\n");
    write_file(P + "badnode.csv", "node_id,f0\n0,1.5\nq,2.5\n");
    write_file(P + "negnode.csv", "0,1.5\n-1,2.5\n");
    write_file(P + "badfeat.csv", "0,1.5,2\n1,abc,2\n");
    write_file(P + "nofeat.csv", "0\n1\n");
    write_file(P + "ragged.csv", "0,1,2,3\n1,1,2\n");
    write_file(P + "edges_ok.csv", "0,1\n1,0\n");

    const std::vector<Case> cases = {
        // -- tensor.cpp ------------------------------------------------------
        {"tensor.cpp:29 dense size", false,
         [] { Tensor::dense(2, 3, std::vector<float>(5, 0.f)); }},
        {"tensor.cpp:47 csr row_ptr size", false,
         [] { Tensor::sparse_csr(2, 2, {0, 1}, {0}, {1.f}); }},
        {"tensor.cpp:53 csr col_ind vs values", false,
         [] { Tensor::sparse_csr(2, 2, {0, 1, 1}, {0}, {1.f, 2.f}); }},
        {"tensor.cpp:61 csr row_ptr.back", false,
         [] { Tensor::sparse_csr(2, 2, {0, 1, 3}, {0, 1}, {1.f, 2.f}); }},
        {"tensor.cpp:70 csr col_ind too large", false,
         [] { Tensor::sparse_csr(2, 2, {0, 1, 2}, {0, 2}, {1.f, 1.f}); }},
        {"tensor.cpp:70 csr col_ind negative", false,
         [] { Tensor::sparse_csr(2, 2, {0, 1, 2}, {-1, 0}, {1.f, 1.f}); }},
        {"tensor.cpp:79 csr row_ptr decreasing", false,
         [] { Tensor::sparse_csr(3, 3, {0, 2, 1, 2}, {0, 1}, {1.f, 1.f}); }},
        {"tensor.cpp:133 at() const on CSR", false,
         [] {
             const Tensor t = csr3();
             (void)t.at(0, 0);
         }},
        {"tensor.cpp:137 at() const out of range", false,
         [] {
             const Tensor t = dn(2, 2);
             (void)t.at(2, 0);
         }},
        {"tensor.cpp:148 at() on CSR", false,
         [] {
             Tensor t = csr3();
             t.at(0, 0) = 1.f;
         }},
        {"tensor.cpp:152 at() out of range", false,
         [] {
             Tensor t = dn(2, 2);
             t.at(0, 5) = 1.f;
         }},
        // -- ops.cpp -----------------------------------------------------------
        {"ops.cpp:74 matmul A CSR", false, [] { matmul(csr3(), dn(3, 2)); }},
        {"ops.cpp:79 matmul B CSR", false, [] { matmul(dn(2, 3), csr3()); }},
        {"ops.cpp:91 matmul dims", false, [] { matmul(dn(2, 3), dn(4, 2)); }},
        {"ops.cpp:202 spmm A dense", false, [] { spmm(dn(3, 3), dn(3, 2)); }},
        {"ops.cpp:209 spmm B CSR", false, [] { spmm(csr3(), csr3()); }},
        {"ops.cpp:221 spmm dims", false, [] { spmm(csr3(), dn(4, 2)); }},
        {"ops.cpp:306 relu_inplace CSR", false,
         [] {
             Tensor t = csr3();
             relu_inplace(t);
         }},
        {"ops.cpp:306 leaky_relu_inplace CSR", false,
         [] {
             Tensor t = csr3();
             leaky_relu_inplace(t);
         }},
        {"ops.cpp:306 elu_inplace CSR", false,
         [] {
             Tensor t = csr3();
             elu_inplace(t);
         }},
        {"ops.cpp:306 sigmoid_inplace CSR", false,
         [] {
             Tensor t = csr3();
             sigmoid_inplace(t);
         }},
        {"ops.cpp:306 tanh_inplace CSR", false,
         [] {
             Tensor t = csr3();
             tanh_inplace(t);
         }},
        {"ops.cpp:306 gelu_inplace CSR", false,
         [] {
             Tensor t = csr3();
             gelu_inplace(t);
         }},
        {"ops.cpp:306 softmax_inplace CSR", false,
         [] {
             Tensor t = csr3();
             softmax_inplace(t);
         }},
        {"ops.cpp:306 log_softmax_inplace CSR", false,
         [] {
             Tensor t = csr3();
             log_softmax_inplace(t);
         }},
        {"ops.cpp:306 add_bias X CSR", false,
         [] {
             Tensor t = csr3();
             add_bias(t, dn(1, 3));
         }},
        {"ops.cpp:513 softmax 0 columns", false,
         [] {
             Tensor t = dn(2, 0);
             softmax_inplace(t);
         }},
        {"ops.cpp:572 log_softmax 0 columns", false,
         [] {
             Tensor t = dn(2, 0);
             log_softmax_inplace(t);
         }},
        {"ops.cpp:626 add_bias bias CSR", false,
         [] {
             Tensor t = dn(3, 3);
             add_bias(t, csr3());
         }},
        {"ops.cpp:634 add_bias shape", false,
         [] {
             Tensor t = dn(2, 3);
             add_bias(t, dn(1, 2));
         }},
        // -- layers.cpp --------------------------------------------------------
        {"layers.cpp:46 add_self_loops dense", false, [] { add_self_loops(dn(3, 3)); }},
        {"layers.cpp:50 add_self_loops not square", false, [] { add_self_loops(csr23()); }},
        {"layers.cpp:46 gcn_norm dense", false, [] { gcn_norm(dn(3, 3)); }},
        {"layers.cpp:50 gcn_norm not square", false, [] { gcn_norm(csr23()); }},
        {"layers.cpp:223 GCNLayer in_features 0", false, [] { GCNLayer l(0, 4); }},
        {"layers.cpp:227 GCNLayer out_features 0", false, [] { GCNLayer l(4, 0); }},
        {"layers.cpp:237 GCNLayer::set_weight CSR", false,
         [] {
             GCNLayer l(3, 3);
             l.set_weight(csr3());
         }},
        {"layers.cpp:241 GCNLayer::set_weight shape", false,
         [] {
             GCNLayer l(3, 4);
             l.set_weight(dn(4, 3));
         }},
        {"layers.cpp:256 GCNLayer::set_bias without bias", false,
         [] {
             GCNLayer l(3, 4, false);
             l.set_bias(dn(1, 4));
         }},
        {"layers.cpp:260 GCNLayer::set_bias CSR", false,
         [] {
             GCNLayer l(3, 3);
             l.set_bias(csr3());
         }},
        {"layers.cpp:264 GCNLayer::set_bias shape", false,
         [] {
             GCNLayer l(3, 4);
             l.set_bias(dn(1, 3));
         }},
        {"layers.cpp:289 GCNLayer::forward A dense", false,
         [] { GCNLayer(3, 2).forward(dn(3, 3), dn(3, 3)); }},
        {"layers.cpp:294 GCNLayer::forward A not square", false,
         [] { GCNLayer(3, 2).forward(csr23(), dn(2, 3)); }},
        {"layers.cpp:302 GCNLayer::forward H CSR", false,
         [] { GCNLayer(3, 2).forward(csr3(), csr3()); }},
        {"layers.cpp:306 GCNLayer::forward H columns", false,
         [] { GCNLayer(4, 2).forward(csr3(), dn(3, 3)); }},
        {"layers.cpp:312 GCNLayer::forward rows", false,
         [] { GCNLayer(3, 2).forward(csr3(), dn(4, 3)); }},
        {"layers.cpp:361 sage_max_aggregate A dense", false,
         [] { sage_max_aggregate(dn(3, 3), dn(3, 2)); }},
        {"layers.cpp:365 sage_max_aggregate H CSR", false,
         [] { sage_max_aggregate(csr3(), csr3()); }},
        {"layers.cpp:369 sage_max_aggregate rows", false,
         [] { sage_max_aggregate(csr3(), dn(4, 2)); }},
        {"layers.cpp:452 SAGELayer in_features 0", false, [] { SAGELayer l(0, 4); }},
        {"layers.cpp:456 SAGELayer out_features 0", false, [] { SAGELayer l(4, 0); }},
        {"layers.cpp:466 SAGELayer::set_weight_neigh CSR", false,
         [] {
             SAGELayer l(3, 3);
             l.set_weight_neigh(csr3());
         }},
        {"layers.cpp:470 SAGELayer::set_weight_neigh shape", false,
         [] {
             SAGELayer l(3, 4);
             l.set_weight_neigh(dn(3, 3));
         }},
        {"layers.cpp:485 SAGELayer::set_weight_self CSR", false,
         [] {
             SAGELayer l(3, 3);
             l.set_weight_self(csr3());
         }},
        {"layers.cpp:489 SAGELayer::set_weight_self shape", false,
         [] {
             SAGELayer l(3, 4);
             l.set_weight_self(dn(4, 4));
         }},
        {"layers.cpp:504 SAGELayer::set_bias without bias", false,
         [] {
             SAGELayer l(3, 4, SAGELayer::Aggregator::Mean, false);
             l.set_bias(dn(1, 4));
         }},
        {"layers.cpp:508 SAGELayer::set_bias CSR", false,
         [] {
             SAGELayer l(3, 3);
             l.set_bias(csr3());
         }},
        {"layers.cpp:512 SAGELayer::set_bias shape", false,
         [] {
             SAGELayer l(3, 4);
             l.set_bias(dn(2, 4));
         }},
        {"layers.cpp:541 SAGELayer::forward A dense", false,
         [] { SAGELayer(3, 2).forward(dn(3, 3), dn(3, 3)); }},
        {"layers.cpp:547 SAGELayer::forward H CSR", false,
         [] { SAGELayer(3, 2).forward(csr3(), csr3()); }},
        {"layers.cpp:551 SAGELayer::forward H columns", false,
         [] { SAGELayer(5, 2).forward(csr3(), dn(3, 3)); }},
        {"layers.cpp:557 SAGELayer::forward A.cols vs H.rows", false,
         [] { SAGELayer(3, 2).forward(csr23(), dn(2, 3)); }},
        {"layers.cpp:770 edge_softmax dense", false, [] { edge_softmax(dn(3, 3)); }},
        {"layers.cpp:840 GATLayer in_features 0", false, [] { GATLayer l(0, 4); }},
        {"layers.cpp:844 GATLayer out_features 0", false, [] { GATLayer l(4, 0); }},
        {"layers.cpp:854 GATLayer::set_weight CSR", false,
         [] {
             GATLayer l(3, 3);
             l.set_weight(csr3());
         }},
        {"layers.cpp:858 GATLayer::set_weight shape", false,
         [] {
             GATLayer l(3, 4);
             l.set_weight(dn(3, 5));
         }},
        {"layers.cpp:873 GATLayer::set_attn_left CSR", false,
         [] {
             GATLayer l(3, 3);
             l.set_attn_left(csr3());
         }},
        {"layers.cpp:877 GATLayer::set_attn_left shape", false,
         [] {
             GATLayer l(3, 4);
             l.set_attn_left(dn(4, 1));
         }},
        {"layers.cpp:891 GATLayer::set_attn_right CSR", false,
         [] {
             GATLayer l(3, 3);
             l.set_attn_right(csr3());
         }},
        {"layers.cpp:895 GATLayer::set_attn_right shape", false,
         [] {
             GATLayer l(3, 4);
             l.set_attn_right(dn(1, 3));
         }},
        {"layers.cpp:909 GATLayer::set_bias without bias", false,
         [] {
             GATLayer l(3, 4, 0.2f, false);
             l.set_bias(dn(1, 4));
         }},
        {"layers.cpp:913 GATLayer::set_bias CSR", false,
         [] {
             GATLayer l(3, 3);
             l.set_bias(csr3());
         }},
        {"layers.cpp:917 GATLayer::set_bias shape", false,
         [] {
             GATLayer l(3, 4);
             l.set_bias(dn(1, 5));
         }},
        {"layers.cpp:948 GATLayer::forward A dense", false,
         [] { GATLayer(3, 2).forward(dn(3, 3), dn(3, 3)); }},
        {"layers.cpp:953 GATLayer::forward A not square", false,
         [] { GATLayer(3, 2).forward(csr23(), dn(2, 3)); }},
        {"layers.cpp:960 GATLayer::forward H CSR", false,
         [] { GATLayer(3, 2).forward(csr3(), csr3()); }},
        {"layers.cpp:964 GATLayer::forward H columns", false,
         [] { GATLayer(2, 2).forward(csr3(), dn(3, 3)); }},
        {"layers.cpp:970 GATLayer::forward rows", false,
         [] { GATLayer(3, 2).forward(csr3(), dn(5, 3)); }},
        // -- model.cpp ---------------------------------------------------------
        {"model.cpp:34 load_cora_binary truncated", false,
         [&] { load_cora_binary(P + "short.cora"); }},
        {"model.cpp:34 load_weight_file truncated", false,
         [&] { load_weight_file(P + "short.tgnn"); }},
        {"model.cpp:52 load_cora_binary cannot open", false,
         [&] { load_cora_binary(P + "missing.cora"); }},
        {"model.cpp:137 load_weight_file cannot open", false,
         [&] { load_weight_file(P + "missing.tgnn"); }},
        {"model.cpp:146 load_weight_file magic", false,
         [&] { load_weight_file(P + "magic.tgnn"); }},
        {"model.cpp:153 load_weight_file version", false,
         [&] { load_weight_file(P + "version.tgnn"); }},
        // (this build's layers hold their zero weights on the device from
        // add_*_layer on, as the reference's hold them on the host)
        {"model.cpp:262 Model::load_weights missing tensor", true,
         [] {
             Model m;
             m.add_gcn_layer(3, 2);
             WeightFile wf;  // the first tensor load_weights reads is missing
             wf.tensors["layer0.bias"] = dn(1, 2);
             m.load_weights(wf);
         }},
        {"model.cpp:361 Model::forward no layers", false,
         [] {
             Model m;
             m.forward(csr3(), dn(3, 3));
         }},
        // -- graph_loader.cpp (this build parses on the device) ---------------
        {"graph_loader.cpp:41 parse_edges cannot open", false,
         [&] { GraphLoader::parse_edges(P + "missing.csv"); }},
        {"graph_loader.cpp:41 parse_features cannot open", false,
         [&] { GraphLoader::parse_features(P + "missing.csv"); }},
        {"graph_loader.cpp:65 parse_edges empty", true,
         [&] { GraphLoader::parse_edges(P + "empty.csv"); }},
        {"graph_loader.cpp:78 parse_edges malformed line", true,
         [&] { GraphLoader::parse_edges(P + "nocomma.csv"); }},
        {"graph_loader.cpp:89 parse_edges invalid integer", true,
         [&] { GraphLoader::parse_edges(P + "badint.csv"); }},
        {"graph_loader.cpp:95 parse_edges negative id", true,
         [&] { GraphLoader::parse_edges(P + "negid.csv"); }},
        {"graph_loader.cpp:113 parse_features empty", true,
         [&] { GraphLoader::parse_features(P + "empty.csv"); }},
        {"graph_loader.cpp:120 parse_features no data rows", true,
         [&] { GraphLoader::parse_features(P + "header_only.csv"); }},
        {"graph_loader.cpp:151 parse_features invalid node_id", true,
         [&] { GraphLoader::parse_features(P + "badnode.csv"); }},
        {"graph_loader.cpp:156 parse_features negative node_id", true,
         [&] { GraphLoader::parse_features(P + "negnode.csv"); }},
        {"graph_loader.cpp:168 parse_features invalid feature", true,
         [&] { GraphLoader::parse_features(P + "badfeat.csv"); }},
        {"graph_loader.cpp:178 parse_features no features", true,
         [&] { GraphLoader::parse_features(P + "nofeat.csv"); }},
        {"graph_loader.cpp:183 parse_features inconsistent count", true,
         [&] { GraphLoader::parse_features(P + "ragged.csv"); }},
        {"graph_loader.cpp:218 edge_list_to_csr 0 nodes", false,
         [] { GraphLoader::edge_list_to_csr({{0, 0}}, 0); }},
        {"graph_loader.cpp:231 edge_list_to_csr src range", true,
         [] { GraphLoader::edge_list_to_csr({{0, 1}, {3, 0}}, 3); }},
        {"graph_loader.cpp:237 edge_list_to_csr dst range", true,
         [] { GraphLoader::edge_list_to_csr({{0, 1}, {1, -1}}, 3); }},
        {"graph_loader.cpp:65 load (edges empty)", true,
         [&] { GraphLoader::load(P + "empty.csv", P + "ragged.csv"); }},
        {"graph_loader.cpp:183 load (features ragged)", true,
         [&] { GraphLoader::load(P + "edges_ok.csv", P + "ragged.csv"); }},
    };
    for (const Case& c : cases)
        if (mode == "all" || !c.device) run(c);
    return 0;
}
