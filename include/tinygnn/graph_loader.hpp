// tinygnn/graph_loader.hpp -- graph ingestion of TinyGNN's API (reference
// include/tinygnn/graph_loader.hpp:17-89), running on the device.
//
// The files are read into HBM and parsed there (the C-ABI's tg_csv_*):
// line splitting, header detection, std::stoi / std::stof conversions and
// error messages are the reference's, and the results are device-resident
// tensors (host views copy back on access).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "tinygnn/tensor.hpp"

namespace tinygnn {

/// The loaded graph (graph_loader.hpp:17-23).
struct GraphData {
    Tensor adjacency;      // SparseCSR num_nodes x num_nodes, values 1.0
    Tensor node_features;  // Dense num_nodes x num_features
    std::size_t num_nodes = 0;
    std::size_t num_edges = 0;
    std::size_t num_features = 0;
};

struct GraphLoader {
    /// Edge-list CSV -> (src, dst) pairs (graph_loader.cpp:61-107): optional
    /// header row, LF or CRLF, blank lines skipped.  std::runtime_error on an
    /// unreadable or empty file, a line without ',', a non-integer or a
    /// negative id, naming the line.
    static std::vector<std::pair<int32_t, int32_t>> parse_edges(const std::string& path);

    /// Node-feature CSV -> Dense (max node_id + 1) x num_features, rows
    /// placed by node_id, missing ids zero (graph_loader.cpp:112-206).
    static Tensor parse_features(const std::string& path);

    /// Edge list (src, dst) -> num_nodes x num_nodes CSR, row = src, each row's
    /// destinations sorted ascending, duplicates kept, values 1.0f
    /// (graph_loader.cpp:211-281).  Bit-identical; the result is
    /// device-resident.  Out-of-range endpoints throw std::invalid_argument
    /// naming the first bad edge.
    static Tensor edge_list_to_csr(const std::vector<std::pair<int32_t, int32_t>>& edges,
                                   std::size_t num_nodes);

    /// Both files -> GraphData (graph_loader.cpp:286-326): num_nodes = the
    /// larger of (largest endpoint + 1) and the feature rows; features are
    /// zero-padded to num_nodes rows.  Edges and CSR never leave the device.
    static GraphData load(const std::string& edges_path, const std::string& features_path);
};

/// The SparseCSR num_nodes x num_nodes adjacency of a COO edge list as the
/// pybind module's Tensor.from_edge_index builds it (python/tinygnn_ext.cpp:
/// 116-157): rows = sources, destinations sorted, duplicates kept, values
/// 1.0f, destinations checked by Tensor::sparse_csr's validation.  A source
/// outside [0, num_nodes) (undefined behaviour in the reference) throws
/// std::invalid_argument.  src / dst are host arrays of num_edges entries.
Tensor csr_from_edge_index(const int32_t* src, const int32_t* dst, std::size_t num_edges,
                           std::size_t num_nodes);

}  // namespace tinygnn
