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

#include "tinygnn/layers.hpp"
#include "tinygnn/tensor.hpp"

namespace tinygnn {

/// Named weight tensors (model.hpp:76-79).
struct WeightFile {
    float test_accuracy = 0.0f;
    std::unordered_map<std::string, Tensor> tensors;
};

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

    /// Full execution graph on the device (model.cpp:359-439).
    Tensor forward(const Tensor& adjacency, const Tensor& features) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    std::size_t num_layers_ = 0;
};

}  // namespace tinygnn
