// tinygnn/graph_loader.hpp -- CSR construction of TinyGNN's API (reference
// include/tinygnn/graph_loader.hpp:74-76), built on the device.
#pragma once

#include <cstddef>
#include <cstdint>
#include <utility>
#include <vector>

#include "tinygnn/tensor.hpp"

namespace tinygnn {

struct GraphLoader {
    /// Edge list (src, dst) -> num_nodes x num_nodes CSR, row = src, each row's
    /// destinations sorted ascending, duplicates kept, values 1.0f
    /// (graph_loader.cpp:211-281).  Bit-identical; the result is
    /// device-resident.  Out-of-range endpoints throw std::invalid_argument
    /// naming the first bad edge.
    static Tensor edge_list_to_csr(const std::vector<std::pair<int32_t, int32_t>>& edges,
                                   std::size_t num_nodes);
};

}  // namespace tinygnn
