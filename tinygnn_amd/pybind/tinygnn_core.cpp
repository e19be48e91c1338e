// tinygnn_core.cpp -- the Python module `_tinygnn_core`: the binding surface
// of the reference's pybind module (python/tinygnn_ext.cpp:179-452) -- same
// module name, classes, functions, argument names and defaults -- over this
// build's C++ API (include/tinygnn/*.hpp), whose tensors live in HBM.
//
// Conversions keep the reference's contract: from_numpy / from_scipy_csr /
// from_edge_index copy their input, to_numpy and the *_numpy accessors
// return copies, errors are std::invalid_argument -> ValueError,
// std::out_of_range -> IndexError, std::runtime_error -> RuntimeError.
// Added for the device: a Dense tensor exposes __cuda_array_interface__ (its
// HBM buffer, zero-copy, for torch.as_tensor and other consumers), a CSR
// tensor exposes its three buffers through device_arrays(), and
// Tensor._from_device copies a device buffer into a new tensor.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tinygnn/graph_loader.hpp"
#include "tinygnn/layers.hpp"
#include "tinygnn/model.hpp"
#include "tinygnn/ops.hpp"
#include "tinygnn/tensor.hpp"

namespace py = pybind11;
using namespace tinygnn;

namespace {

using FloatArray = py::array_t<float, py::array::c_style | py::array::forcecast>;
using IntArray = py::array_t<int32_t, py::array::c_style | py::array::forcecast>;

Tensor dense_of(const FloatArray& a, const char* who) {
    const py::buffer_info b = a.request();
    if (b.ndim != 2)
        throw std::invalid_argument(std::string(who) + ": expected 2D array, got " +
                                    std::to_string(b.ndim) + "D");
    const auto rows = static_cast<std::size_t>(b.shape[0]);
    const auto cols = static_cast<std::size_t>(b.shape[1]);
    const float* p = static_cast<const float*>(b.ptr);
    return Tensor::dense(rows, cols, std::vector<float>(p, p + rows * cols));
}

Tensor dense_of_1d(const FloatArray& a) {
    const py::buffer_info b = a.request();
    if (b.ndim == 1) {
        const auto cols = static_cast<std::size_t>(b.shape[0]);
        const float* p = static_cast<const float*>(b.ptr);
        return Tensor::dense(1, cols, std::vector<float>(p, p + cols));
    }
    if (b.ndim == 2) return dense_of(a, "Tensor.from_numpy_1d");
    throw std::invalid_argument("Tensor.from_numpy_1d: expected 1D or 2D array, got " +
                                std::to_string(b.ndim) + "D");
}

py::array_t<float> to_numpy(const Tensor& t) {
    if (t.format() != StorageFormat::Dense)
        throw std::invalid_argument("to_numpy: only Dense tensors can be converted to NumPy.");
    py::array_t<float> out({static_cast<py::ssize_t>(t.rows()), static_cast<py::ssize_t>(t.cols())});
    const std::vector<float>& d = t.data();
    std::copy(d.begin(), d.end(), static_cast<float*>(out.request().ptr));
    return out;
}

template <typename T>
py::array_t<T> vec_copy(const std::vector<T>& v) {
    py::array_t<T> out(static_cast<py::ssize_t>(v.size()));
    std::copy(v.begin(), v.end(), static_cast<T*>(out.request().ptr));
    return out;
}

Tensor from_scipy_csr(const py::object& m) {
    const auto shape = m.attr("shape").cast<py::tuple>();
    const auto rows = shape[0].cast<std::size_t>();
    const auto cols = shape[1].cast<std::size_t>();
    const IntArray indptr = m.attr("indptr").cast<IntArray>();
    const IntArray indices = m.attr("indices").cast<IntArray>();
    const FloatArray data = m.attr("data").cast<FloatArray>();
    const int32_t* rp = indptr.data();
    const auto nnz = static_cast<std::size_t>(rp[rows]);
    return Tensor::sparse_csr(rows, cols, std::vector<int32_t>(rp, rp + rows + 1),
                              std::vector<int32_t>(indices.data(), indices.data() + nnz),
                              std::vector<float>(data.data(), data.data() + nnz));
}

Tensor from_edge_index(const IntArray& ei, std::size_t num_nodes) {
    const py::buffer_info b = ei.request();
    if (b.ndim != 2 || b.shape[0] != 2)
        throw std::invalid_argument("from_edge_index: expected shape (2, E), got (" +
                                    std::to_string(b.shape[0]) + ", " +
                                    std::to_string(b.ndim > 1 ? b.shape[1] : 0) + ")");
    const auto e = static_cast<std::size_t>(b.shape[1]);
    const int32_t* p = static_cast<const int32_t*>(b.ptr);
    return csr_from_edge_index(p, p + e, e, num_nodes);
}

py::dict array_interface(std::uintptr_t ptr, std::vector<py::ssize_t> shape, const char* typestr) {
    py::dict d;
    d["shape"] = py::tuple(py::cast(shape));
    d["typestr"] = typestr;
    d["data"] = py::make_tuple(ptr, false);
    d["version"] = 2;
    d["strides"] = py::none();
    return d;
}

}  // namespace

PYBIND11_MODULE(_tinygnn_core, m) {
    m.doc() = "TinyGNN on MI355X: the reference's Python API over HIP kernels";

    py::enum_<StorageFormat>(m, "StorageFormat")
        .value("Dense", StorageFormat::Dense)
        .value("SparseCSR", StorageFormat::SparseCSR)
        .export_values();
    py::enum_<Activation>(m, "Activation")
        .value("NONE", Activation::None)
        .value("RELU", Activation::ReLU)
        .export_values();

    py::class_<Tensor>(m, "Tensor")
        .def(py::init<>(), "An empty 0x0 Dense tensor")
        .def_static("dense", py::overload_cast<std::size_t, std::size_t>(&Tensor::dense),
                    "Zero-filled Dense tensor", py::arg("rows"), py::arg("cols"))
        .def_static("dense_from_data",
                    [](std::size_t rows, std::size_t cols, std::vector<float> data) {
                        return Tensor::dense(rows, cols, std::move(data));
                    },
                    "Dense tensor from row-major data", py::arg("rows"), py::arg("cols"),
                    py::arg("data"))
        .def_static("sparse_csr", &Tensor::sparse_csr, "SparseCSR tensor (validated)",
                    py::arg("rows"), py::arg("cols"), py::arg("row_ptr"), py::arg("col_ind"),
                    py::arg("values"))
        .def_static("from_numpy", [](const FloatArray& a) { return dense_of(a, "Tensor.from_numpy"); },
                    "Dense tensor from a 2-D array (copied, cast to float32)", py::arg("array"))
        .def_static("from_numpy_1d", &dense_of_1d, "Dense 1xN (1-D input) or 2-D tensor",
                    py::arg("array"))
        .def_static("from_scipy_csr", &from_scipy_csr, "SparseCSR tensor from a scipy csr_matrix",
                    py::arg("csr_matrix"))
        .def_static("from_edge_index", &from_edge_index,
                    "SparseCSR adjacency from a (2, E) edge_index (built on the device)",
                    py::arg("edge_index"), py::arg("num_nodes"))
        .def_static("_from_device",
                    [](std::size_t rows, std::size_t cols, std::uintptr_t ptr) {
                        return Tensor::dense_from_device(rows, cols,
                                                         reinterpret_cast<const float*>(ptr));
                    },
                    py::arg("rows"), py::arg("cols"), py::arg("device_ptr"))
        .def("to_numpy", &to_numpy, "Dense tensor as a NumPy array (copy)")
        .def("row_ptr_numpy", [](const Tensor& t) { return vec_copy(t.row_ptr()); })
        .def("col_ind_numpy", [](const Tensor& t) { return vec_copy(t.col_ind()); })
        .def("values_numpy", [](const Tensor& t) { return vec_copy(t.data()); })
        .def_property_readonly("format", &Tensor::format)
        .def_property_readonly("rows", &Tensor::rows)
        .def_property_readonly("cols", &Tensor::cols)
        .def_property_readonly("numel", &Tensor::numel)
        .def_property_readonly("nnz", &Tensor::nnz)
        .def_property_readonly("memory_footprint_bytes", &Tensor::memory_footprint_bytes)
        .def("at", py::overload_cast<std::size_t, std::size_t>(&Tensor::at, py::const_),
             py::arg("row"), py::arg("col"))
        .def("repr", &Tensor::repr)
        .def("__repr__", &Tensor::repr)
        .def_property_readonly(
            "__cuda_array_interface__",
            [](Tensor& t) {
                if (t.format() != StorageFormat::Dense)
                    throw py::attribute_error("__cuda_array_interface__: Dense tensors only; "
                                              "use device_arrays() for SparseCSR");
                const auto p = reinterpret_cast<std::uintptr_t>(t.device_data_mutable());
                return array_interface(p, {static_cast<py::ssize_t>(t.rows()),
                                            static_cast<py::ssize_t>(t.cols())}, "<f4");
            })
        .def("device_arrays",
             [](const Tensor& t) {
                 if (t.format() != StorageFormat::SparseCSR)
                     throw std::invalid_argument("device_arrays: SparseCSR tensors only");
                 const auto n = static_cast<py::ssize_t>(t.rows());
                 const auto z = static_cast<py::ssize_t>(t.nnz());
                 return py::make_tuple(
                     array_interface(reinterpret_cast<std::uintptr_t>(t.device_row_ptr()), {n + 1}, "<i4"),
                     array_interface(reinterpret_cast<std::uintptr_t>(t.device_col_ind()), {z}, "<i4"),
                     array_interface(reinterpret_cast<std::uintptr_t>(t.device_data()), {z}, "<f4"));
             },
             "(row_ptr, col_ind, values) device buffer descriptions (CUDA array interface)");

    m.def("matmul", &matmul, "C = A x B (Dense)", py::arg("A"), py::arg("B"));
    m.def("spmm", static_cast<Tensor (*)(const Tensor&, const Tensor&)>(&spmm),
          "C = A x B (SparseCSR x Dense)", py::arg("A"), py::arg("B"));
    m.def("relu_inplace", &relu_inplace, py::arg("X"));
    m.def("leaky_relu_inplace", &leaky_relu_inplace, py::arg("X"), py::arg("alpha") = 0.01f);
    m.def("elu_inplace", &elu_inplace, py::arg("X"), py::arg("alpha") = 1.0f);
    m.def("sigmoid_inplace", &sigmoid_inplace, py::arg("X"));
    m.def("tanh_inplace", &tanh_inplace, py::arg("X"));
    m.def("gelu_inplace", &gelu_inplace, py::arg("X"));
    m.def("softmax_inplace", &softmax_inplace, py::arg("X"));
    m.def("log_softmax_inplace", &log_softmax_inplace, py::arg("X"));
    m.def("add_bias", &add_bias, py::arg("X"), py::arg("bias"));

    m.def("add_self_loops", &add_self_loops, py::arg("A"));
    m.def("gcn_norm", &gcn_norm, py::arg("A"));
    m.def("edge_softmax", &edge_softmax, py::arg("A"));
    m.def("sage_max_aggregate", &sage_max_aggregate, py::arg("A"), py::arg("H"));

    py::class_<GCNLayer>(m, "GCNLayer")
        .def(py::init<std::size_t, std::size_t, bool, Activation>(), py::arg("in_features"),
             py::arg("out_features"), py::arg("use_bias") = true,
             py::arg("activation") = Activation::ReLU)
        .def("set_weight", &GCNLayer::set_weight, py::arg("w"))
        .def("set_bias", &GCNLayer::set_bias, py::arg("b"))
        .def("forward", &GCNLayer::forward, py::arg("A_norm"), py::arg("H"))
        .def_property_readonly("in_features", &GCNLayer::in_features)
        .def_property_readonly("out_features", &GCNLayer::out_features)
        .def_property_readonly("has_bias", &GCNLayer::has_bias)
        .def_property_readonly("activation", &GCNLayer::activation)
        .def_property_readonly("weight", &GCNLayer::weight)
        .def_property_readonly("bias", &GCNLayer::bias);

    py::class_<SAGELayer> sage(m, "SAGELayer");
    py::enum_<SAGELayer::Aggregator>(sage, "Aggregator")
        .value("Mean", SAGELayer::Aggregator::Mean)
        .value("Max", SAGELayer::Aggregator::Max)
        .export_values();
    sage.def(py::init<std::size_t, std::size_t, SAGELayer::Aggregator, bool, Activation>(),
             py::arg("in_features"), py::arg("out_features"),
             py::arg("aggregator") = SAGELayer::Aggregator::Mean, py::arg("use_bias") = true,
             py::arg("activation") = Activation::ReLU)
        .def("set_weight_neigh", &SAGELayer::set_weight_neigh, py::arg("w"))
        .def("set_weight_self", &SAGELayer::set_weight_self, py::arg("w"))
        .def("set_bias", &SAGELayer::set_bias, py::arg("b"))
        .def("forward", &SAGELayer::forward, py::arg("A"), py::arg("H"))
        .def_property_readonly("in_features", &SAGELayer::in_features)
        .def_property_readonly("out_features", &SAGELayer::out_features)
        .def_property_readonly("has_bias", &SAGELayer::has_bias)
        .def_property_readonly("activation", &SAGELayer::activation)
        .def_property_readonly("aggregator", &SAGELayer::aggregator)
        .def_property_readonly("weight_neigh", &SAGELayer::weight_neigh)
        .def_property_readonly("weight_self", &SAGELayer::weight_self)
        .def_property_readonly("bias", &SAGELayer::bias);

    py::class_<GATLayer>(m, "GATLayer")
        .def(py::init<std::size_t, std::size_t, float, bool, Activation>(),
             py::arg("in_features"), py::arg("out_features"), py::arg("negative_slope") = 0.2f,
             py::arg("use_bias") = true, py::arg("activation") = Activation::None)
        .def("set_weight", &GATLayer::set_weight, py::arg("w"))
        .def("set_attn_left", &GATLayer::set_attn_left, py::arg("a"))
        .def("set_attn_right", &GATLayer::set_attn_right, py::arg("a"))
        .def("set_bias", &GATLayer::set_bias, py::arg("b"))
        .def("forward", &GATLayer::forward, py::arg("A"), py::arg("H"))
        .def_property_readonly("in_features", &GATLayer::in_features)
        .def_property_readonly("out_features", &GATLayer::out_features)
        .def_property_readonly("negative_slope", &GATLayer::negative_slope)
        .def_property_readonly("has_bias", &GATLayer::has_bias)
        .def_property_readonly("activation", &GATLayer::activation)
        .def_property_readonly("weight", &GATLayer::weight)
        .def_property_readonly("attn_left", &GATLayer::attn_left)
        .def_property_readonly("attn_right", &GATLayer::attn_right)
        .def_property_readonly("bias", &GATLayer::bias);

    py::class_<Model> model(m, "Model");
    py::enum_<Model::InterActivation>(model, "InterActivation")
        .value("NONE", Model::InterActivation::None)
        .value("RELU", Model::InterActivation::ReLU)
        .value("ELU", Model::InterActivation::ELU)
        .export_values();
    model.def(py::init<>())
        .def("add_gcn_layer", &Model::add_gcn_layer, py::arg("in_f"), py::arg("out_f"),
             py::arg("bias") = true, py::arg("act") = Activation::ReLU,
             py::arg("post") = Model::InterActivation::None)
        .def("add_sage_layer", &Model::add_sage_layer, py::arg("in_f"), py::arg("out_f"),
             py::arg("agg") = SAGELayer::Aggregator::Mean, py::arg("bias") = true,
             py::arg("act") = Activation::ReLU, py::arg("post") = Model::InterActivation::None)
        .def("add_gat_layer", &Model::add_gat_layer, py::arg("in_f"), py::arg("out_f"),
             py::arg("num_heads") = static_cast<std::size_t>(1), py::arg("concat") = true,
             py::arg("neg_slope") = 0.2f, py::arg("bias") = true,
             py::arg("act") = Activation::None, py::arg("post") = Model::InterActivation::None)
        .def("load_weights", py::overload_cast<const std::string&>(&Model::load_weights),
             py::arg("path"))
        .def("load_weights_from_file", py::overload_cast<const WeightFile&>(&Model::load_weights),
             "Load weights from a WeightFile object", py::arg("weight_file"))
        .def("forward", &Model::forward, py::arg("adjacency"), py::arg("features"))
        .def_property_readonly("num_layers", &Model::num_layers);

    py::class_<CoraData>(m, "CoraData")
        .def_readonly("num_nodes", &CoraData::num_nodes)
        .def_readonly("num_features", &CoraData::num_features)
        .def_readonly("num_classes", &CoraData::num_classes)
        .def_readonly("num_edges", &CoraData::num_edges)
        .def_readonly("adjacency", &CoraData::adjacency)
        .def_readonly("features", &CoraData::features)
        .def_readonly("labels", &CoraData::labels)
        .def_readonly("train_mask", &CoraData::train_mask)
        .def_readonly("val_mask", &CoraData::val_mask)
        .def_readonly("test_mask", &CoraData::test_mask);

    py::class_<WeightFile>(m, "WeightFile")
        .def_readonly("test_accuracy", &WeightFile::test_accuracy)
        .def_readonly("tensors", &WeightFile::tensors);

    m.def("load_cora_binary", &load_cora_binary, py::arg("path"));
    m.def("load_weight_file", &load_weight_file, py::arg("path"));

    py::class_<GraphData>(m, "GraphData")
        .def_readonly("adjacency", &GraphData::adjacency)
        .def_readonly("node_features", &GraphData::node_features)
        .def_readonly("num_nodes", &GraphData::num_nodes)
        .def_readonly("num_edges", &GraphData::num_edges)
        .def_readonly("num_features", &GraphData::num_features);

    py::class_<GraphLoader>(m, "GraphLoader")
        .def_static("parse_edges", &GraphLoader::parse_edges, py::arg("path"))
        .def_static("parse_features", &GraphLoader::parse_features, py::arg("path"))
        .def_static("edge_list_to_csr", &GraphLoader::edge_list_to_csr, py::arg("edges"),
                    py::arg("num_nodes"))
        .def_static("load", &GraphLoader::load, py::arg("edges_path"), py::arg("features_path"));

    // The reference sizes its OpenMP pool here; the device path has no host
    // thread pool, so these keep the signature and report one host thread.
    m.def("set_num_threads", [](int) {}, py::arg("n"));
    m.def("get_max_threads", []() { return 1; });
}
