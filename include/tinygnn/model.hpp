// tinygnn/model.hpp -- the sequential GNN execution graph of TinyGNN's API
// (reference include/tinygnn/model.hpp:50-164), running on the MI355X
// through the C-ABI in tinygnn_amd.h (tg_model_*).
//
// forward() keeps the reference's contract: adjacency is the raw CSR without
// self-loops; gcn_norm / add_self_loops are derived inside.  The derived
// adjacency and the row plans are kept between calls while the adjacency
// tensor is the same object at the same version (an in-place edit through
// data() bumps the version and forces the recomputation).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "tinygnn/layers.hpp"
#include "tinygnn/tensor.hpp"

namespace tinygnn {

/// The Cora graph export (model.hpp:50-62).
struct CoraData {
    std::size_t num_nodes = 0;
    std::size_t num_features = 0;
    std::size_t num_classes = 0;
    std::size_t num_edges = 0;
    Tensor adjacency;  // SparseCSR N x N, values 1.0 (device-resident)
    Tensor features;   // Dense N x F (device-resident)
    std::vector<int32_t> labels;
    std::vector<uint8_t> train_mask;
    std::vector<uint8_t> val_mask;
    std::vector<uint8_t> test_mask;
};

/// load_cora_binary (model.cpp:49-129): header, features, labels, masks and
/// the edge list; the adjacency is built on the device.  std::runtime_error
/// on I/O errors (the reference's messages).
CoraData load_cora_binary(const std::string& path);

/// Named weight tensors (model.hpp:76-79).
struct WeightFile {
    float test_accuracy = 0.0f;
    std::unordered_map<std::string, Tensor> tensors;
};

/// load_weight_file (model.cpp:134-185): the TGNN binary format, version 1.
/// std::runtime_error on I/O, magic or version errors.
WeightFile load_weight_file(const std::string& path);

class Model {
public:
    enum class InterActivation : uint8_t {
        None = 0,
        ReLU = 1,
        ELU = 2,
    };

    Model();
    ~Model();
    Model(Model&&) noexcept;
    Model& operator=(Model&&) noexcept;
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    std::size_t add_gcn_layer(std::size_t in_f, std::size_t out_f, bool bias = true,
                              Activation act = Activation::ReLU,
                              InterActivation post = InterActivation::None);
    std::size_t add_sage_layer(std::size_t in_f, std::size_t out_f,
                               SAGELayer::Aggregator agg = SAGELayer::Aggregator::Mean,
                               bool bias = true, Activation act = Activation::ReLU,
                               InterActivation post = InterActivation::None);
    std::size_t add_gat_layer(std::size_t in_f, std::size_t out_f, std::size_t num_heads = 1,
                              bool concat = true, float neg_slope = 0.2f, bool bias = true,
                              Activation act = Activation::None,
                              InterActivation post = InterActivation::None);

    std::size_t num_layers() const noexcept { return num_layers_; }

    /// Maps layer{i}.weight|bias|weight_neigh|weight_self and
    /// layer{i}.head{h}.{weight,attn_left,attn_right,bias} onto the layers
    /// (model.cpp:258-305); a missing name throws std::runtime_error.
    void load_weights(const WeightFile& wf);
    /// load_weights(load_weight_file(path)) (model.cpp:252-255).
    void load_weights(const std::string& path);

    /// Full execution graph on the device (model.cpp:359-439).
    Tensor forward(const Tensor& adjacency, const Tensor& features) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    std::size_t num_layers_ = 0;
};

}  // namespace tinygnn
