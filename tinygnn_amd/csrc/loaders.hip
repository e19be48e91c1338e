// loaders.hip -- the binary file formats of TinyGNN's model layer:
//   * the TGNN weight file, version 1 (load_weight_file, reference
//     src/model.cpp:134-185; format include/tinygnn/model.hpp:22-33):
//       "TGNN", u32 version = 1, f32 test accuracy, u32 tensor count, then
//       per tensor u32 name length, name bytes, u32 rows, u32 cols,
//       f32[rows * cols] row-major; all little endian;
//   * the Cora graph export (load_cora_binary, src/model.cpp:49-129):
//       u32 N, F, C, E; f32 features[N * F]; i32 labels[N]; u8 train[N],
//       val[N], test[N]; i32 src[E]; i32 dst[E].
// Files are read on the host (they are host data in the reference too).
// The graph's features go to the device as they are; its adjacency is built
// on the device by the CSR kernels of graph.hip.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "layers.hpp"

struct tg_weights_s {
    float test_accuracy = 0.0f;
    struct Entry {
        std::string name;
        int64_t rows, cols;
        std::vector<float> data;
    };
    std::vector<Entry> entries;  // file order (a repeated name: the last one wins)
};

struct tg_cora_s {
    int64_t n = 0, f = 0, c = 0, e = 0;
    std::vector<float> features;
    std::vector<int32_t> labels;
    std::vector<uint8_t> train, val, test;
    std::vector<int32_t> src, dst;
};

namespace tg {
namespace {

struct File {
    FILE* f = nullptr;
    int64_t size = 0;
    ~File() {
        if (f) std::fclose(f);
    }
};

// read_exact (model.cpp:30-37): "<ctx>: unexpected end of file or read error."
void read_exact(File& fl, void* buf, int64_t n, const char* ctx) {
    if (n == 0) return;
    const int64_t pos = static_cast<int64_t>(std::ftell(fl.f));
    if (n < 0 || pos < 0 || n > fl.size - pos ||
        std::fread(buf, 1, static_cast<size_t>(n), fl.f) != static_cast<size_t>(n))
        throw std::runtime_error(std::string(ctx) + ": unexpected end of file or read error.");
}

template <typename T>
T read_le(File& fl, const char* ctx) {  // little-endian host (x86-64 / gfx950 hosts)
    T v{};
    read_exact(fl, &v, sizeof(T), ctx);
    return v;
}

// Checks that n more bytes exist before a buffer of that size is allocated
// (a truncated file fails here instead of allocating its header's size).
void require_bytes(File& fl, int64_t n, const char* ctx) {
    const int64_t pos = static_cast<int64_t>(std::ftell(fl.f));
    if (n < 0 || pos < 0 || n > fl.size - pos)
        throw std::runtime_error(std::string(ctx) + ": unexpected end of file or read error.");
}

void open_file(File& fl, const char* path, const std::string& open_msg) {
    fl.f = std::fopen(path ? path : "", "rb");
    if (!fl.f) throw std::runtime_error(open_msg);
    if (std::fseek(fl.f, 0, SEEK_END) != 0) throw std::runtime_error(open_msg);
    fl.size = static_cast<int64_t>(std::ftell(fl.f));
    std::rewind(fl.f);
}

void load_weights_file(const char* path, tg_weights_s& w) {
    const std::string p = path ? path : "";
    const char* ctx = "load_weight_file";
    File fl;
    open_file(fl, path, "load_weight_file: cannot open " + p);
    char magic[4];
    read_exact(fl, magic, 4, ctx);
    if (std::memcmp(magic, "TGNN", 4) != 0)
        throw std::runtime_error("load_weight_file: invalid magic in " + p);
    const uint32_t version = read_le<uint32_t>(fl, ctx);
    if (version != 1)
        throw std::runtime_error("load_weight_file: unsupported version " +
                                 std::to_string(version) + " in " + p);
    w.test_accuracy = read_le<float>(fl, ctx);
    const uint32_t count = read_le<uint32_t>(fl, ctx);
    for (uint32_t t = 0; t < count; ++t) {
        const uint32_t name_len = read_le<uint32_t>(fl, ctx);
        require_bytes(fl, name_len, ctx);
        tg_weights_s::Entry e;
        e.name.assign(name_len, '\0');
        read_exact(fl, name_len ? &e.name[0] : nullptr, name_len, ctx);
        e.rows = read_le<uint32_t>(fl, ctx);
        e.cols = read_le<uint32_t>(fl, ctx);
        const int64_t bytes = e.rows * e.cols * int64_t(sizeof(float));
        require_bytes(fl, bytes, ctx);
        e.data.resize(static_cast<size_t>(e.rows * e.cols));
        read_exact(fl, e.data.data(), bytes, ctx);
        w.entries.push_back(std::move(e));
    }
}

void load_cora(const char* path, tg_cora_s& c) {
    const std::string p = path ? path : "";
    const char* ctx = "load_cora_binary";
    File fl;
    open_file(fl, path, "load_cora_binary: cannot open " + p);
    c.n = read_le<uint32_t>(fl, ctx);
    c.f = read_le<uint32_t>(fl, ctx);
    c.c = read_le<uint32_t>(fl, ctx);
    c.e = read_le<uint32_t>(fl, ctx);
    require_bytes(fl, c.n * c.f * 4, ctx);
    c.features.resize(static_cast<size_t>(c.n * c.f));
    read_exact(fl, c.features.data(), c.n * c.f * 4, ctx);
    require_bytes(fl, c.n * 7, ctx);
    c.labels.resize(static_cast<size_t>(c.n));
    read_exact(fl, c.labels.data(), c.n * 4, ctx);
    c.train.resize(static_cast<size_t>(c.n));
    c.val.resize(static_cast<size_t>(c.n));
    c.test.resize(static_cast<size_t>(c.n));
    read_exact(fl, c.train.data(), c.n, ctx);
    read_exact(fl, c.val.data(), c.n, ctx);
    read_exact(fl, c.test.data(), c.n, ctx);
    require_bytes(fl, c.e * 8, ctx);
    c.src.resize(static_cast<size_t>(c.e));
    c.dst.resize(static_cast<size_t>(c.e));
    read_exact(fl, c.src.data(), c.e * 4, ctx);
    read_exact(fl, c.dst.data(), c.e * 4, ctx);
}

}  // namespace
}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_weights_open(const char* path, tg_weights_t* out) {
    return guard([&] {
        require(out != nullptr, "tg_weights_open: out is null");
        *out = nullptr;
        auto w = std::make_unique<tg_weights_s>();
        tg::load_weights_file(path, *w);
        *out = w.release();
    });
}

int tg_weights_info(tg_weights_t w, int64_t* n_tensors, float* test_accuracy) {
    return guard([&] {
        require(w != nullptr, "tg_weights_info: handle is null");
        if (n_tensors) *n_tensors = static_cast<int64_t>(w->entries.size());
        if (test_accuracy) *test_accuracy = w->test_accuracy;
    });
}

int tg_weights_tensor(tg_weights_t w, int64_t i, const char** name, int64_t* name_len,
                      int64_t* rows, int64_t* cols, const float** data) {
    return guard([&] {
        require(w != nullptr, "tg_weights_tensor: handle is null");
        if (i < 0 || i >= static_cast<int64_t>(w->entries.size()))
            throw std::out_of_range("tg_weights_tensor: index out of range");
        const auto& e = w->entries[static_cast<size_t>(i)];
        if (name) *name = e.name.c_str();
        if (name_len) *name_len = static_cast<int64_t>(e.name.size());
        if (rows) *rows = e.rows;
        if (cols) *cols = e.cols;
        if (data) *data = e.data.data();
    });
}

int tg_weights_destroy(tg_weights_t w) {
    return guard([&] { delete w; });
}

int tg_cora_open(const char* path, tg_cora_t* out) {
    return guard([&] {
        require(out != nullptr, "tg_cora_open: out is null");
        *out = nullptr;
        auto c = std::make_unique<tg_cora_s>();
        tg::load_cora(path, *c);
        *out = c.release();
    });
}

int tg_cora_info(tg_cora_t c, int64_t* num_nodes, int64_t* num_features, int64_t* num_classes,
                 int64_t* num_edges) {
    return guard([&] {
        require(c != nullptr, "tg_cora_info: handle is null");
        if (num_nodes) *num_nodes = c->n;
        if (num_features) *num_features = c->f;
        if (num_classes) *num_classes = c->c;
        if (num_edges) *num_edges = c->e;
    });
}

int tg_cora_host(tg_cora_t c, const int32_t** labels, const uint8_t** train_mask,
                 const uint8_t** val_mask, const uint8_t** test_mask) {
    return guard([&] {
        require(c != nullptr, "tg_cora_host: handle is null");
        if (labels) *labels = c->labels.data();
        if (train_mask) *train_mask = c->train.data();
        if (val_mask) *val_mask = c->val.data();
        if (test_mask) *test_mask = c->test.data();
    });
}

int tg_cora_upload(tg_cora_t c, float* features, int32_t* row_ptr, int32_t* col_ind, float* val,
                   tg_stream_t stream) {
    return guard([&] {
        require(c != nullptr, "tg_cora_upload: handle is null");
        const auto s = static_cast<hipStream_t>(stream);
        require(row_ptr != nullptr, "tg_cora_upload: row_ptr is null");
        require(c->e == 0 || (col_ind && val), "tg_cora_upload: null output");
        require(c->n * c->f == 0 || features, "tg_cora_upload: features is null");
        if (c->n * c->f > 0)
            TG_HIP(hipMemcpyAsync(features, c->features.data(),
                                  static_cast<size_t>(c->n * c->f) * sizeof(float),
                                  hipMemcpyHostToDevice, s));
        tg::DeviceBuffer edges(static_cast<size_t>(std::max<int64_t>(c->e, 1)) * 8);
        int32_t* d_src = edges.as<int32_t>();
        int32_t* d_dst = d_src + c->e;
        if (c->e > 0) {
            TG_HIP(hipMemcpyAsync(d_src, c->src.data(), static_cast<size_t>(c->e) * 4,
                                  hipMemcpyHostToDevice, s));
            TG_HIP(hipMemcpyAsync(d_dst, c->dst.data(), static_cast<size_t>(c->e) * 4,
                                  hipMemcpyHostToDevice, s));
        }
        // model.cpp:89-110 counts only sources below N and then writes through
        // every source (a source outside [0, N) is undefined behaviour there and
        // an error here); destinations are checked afterwards by
        // Tensor::sparse_csr (tensor.cpp:46-86)
        tg::edge_list_to_csr(c->n, c->e, d_src, d_dst, row_ptr, col_ind, val, nullptr, 0, s,
                             /*check_dst=*/false, "load_cora_binary");
        tg::csr_validate(c->n, c->n, c->e, row_ptr, col_ind, s);
        TG_HIP(hipStreamSynchronize(s));
    });
}

int tg_cora_destroy(tg_cora_t c) {
    return guard([&] { delete c; });
}

}  // extern "C"
