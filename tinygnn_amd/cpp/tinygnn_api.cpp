// tinygnn_api.cpp -- TinyGNN's C++ API (tensor / ops / layers / model /
// graph_loader) over the C-ABI of libtinygnn_amd.so.
//
// Everything numeric happens on the device through tg_* calls on the
// default (null) HIP stream, with temporaries from the stream-ordered
// allocator on that stream; this file holds the host-side contract of the
// reference: value-semantics tensors, argument validation with the
// reference's exception types and messages (file:line cited per check), and
// the coherence of host views with the device copies.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tinygnn/graph_loader.hpp"
#include "tinygnn/layers.hpp"
#include "tinygnn/model.hpp"
#include "tinygnn/ops.hpp"
#include "tinygnn/tensor.hpp"
#include "tinygnn_amd.h"

namespace tinygnn {
namespace detail {

[[noreturn]] void hip_fail(hipError_t e, const char* what) {
    throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

void check(int status) {
    if (status == TG_OK) return;
    const std::string msg = tg_last_error();
    if (status == TG_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    if (status == TG_ERR_OUT_OF_RANGE) throw std::out_of_range(msg);
    throw std::runtime_error(msg);
}

// Device buffers come from the stream-ordered allocator on the null stream,
// the stream every op of this API runs on: a buffer released while kernels
// that use it are still queued is only reused by work queued after them, so
// no release waits for the device.  They come from a memory pool of the
// library's own per device (created once, under a lock), which keeps freed
// memory (its release threshold is raised), so a warm loop of ops allocates
// without calling into the driver; the device's default pool, which other
// code in the process may use, keeps its own settings.
hipMemPool_t library_pool() {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static hipMemPool_t pools[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        throw std::runtime_error("device ordinal out of range for the memory pools");
    std::lock_guard<std::mutex> lock(mu);
    if (pools[dev] == nullptr) {
        hipMemPoolProps props{};
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        e = hipMemPoolCreate(&pool, &props);
        if (e != hipSuccess) hip_fail(e, "hipMemPoolCreate");
        uint64_t keep = ~uint64_t(0);
        e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) hip_fail(e, "hipMemPoolSetAttribute");
        pools[dev] = pool;
    }
    return pools[dev];
}

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFreeAsync(p, nullptr);
        p = nullptr;
        n = 0;
    }
    void ensure(size_t bytes) {
        if (bytes <= n && p) return;
        release();
        if (bytes == 0) bytes = 4;
        hipError_t e = hipMallocFromPoolAsync(&p, bytes, library_pool(), nullptr);
        if (e != hipSuccess) hip_fail(e, "hipMallocFromPoolAsync");
        n = bytes;
    }
};

struct DeviceMirror {
    DevBuf data, rp, ci;
    bool valid = false;
    tg_spmm_plan_t plan = nullptr;
    int64_t plan_max_f = -1;
    uint64_t plan_version = ~uint64_t(0);
    ~DeviceMirror() {
        if (plan) tg_spmm_plan_destroy(plan);
    }
};

void h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) hip_fail(e, "hipMemcpy H2D");
}

void d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) hip_fail(e, "hipMemcpy D2H");
}

void d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) hip_fail(e, "hipMemcpy D2D");
}

// Private access for the library's own ops.
struct Access {
    static Tensor make(StorageFormat f, size_t rows, size_t cols, size_t count) {
        Tensor t;
        t.format_ = f;
        t.shape_ = {rows, cols};
        t.strides_ = f == StorageFormat::Dense ? std::vector<size_t>{cols, 1} : std::vector<size_t>{};
        t.count_ = count;
        t.host_valid_ = false;
        t.dev_ = std::make_shared<DeviceMirror>();
        t.dev_->data.ensure(count * sizeof(float));
        if (f == StorageFormat::SparseCSR) {
            t.dev_->rp.ensure((rows + 1) * sizeof(int32_t));
            t.dev_->ci.ensure(count * sizeof(int32_t));
        }
        t.dev_->valid = true;
        return t;
    }
    static void set_count(Tensor& t, size_t count) { t.count_ = count; }
    static std::shared_ptr<DeviceMirror> mirror_ptr(const Tensor& t) {
        t.mirror();
        return t.dev_;
    }
    static int32_t* rp(Tensor& t) { return static_cast<int32_t*>(t.dev_->rp.p); }
    static int32_t* ci(Tensor& t) { return static_cast<int32_t*>(t.dev_->ci.p); }
    static float* val(Tensor& t) { return static_cast<float*>(t.dev_->data.p); }
};

// Row plan of a CSR tensor's structure, kept with its device copy.
tg_spmm_plan_t plan_for(const Tensor& a, int64_t max_f) {
    DeviceMirror& m = a.mirror();
    const int32_t* rp = a.device_row_ptr();
    if (m.plan && m.plan_version == a.version() && m.plan_max_f >= max_f) return m.plan;
    if (m.plan) tg_spmm_plan_destroy(m.plan);
    m.plan = nullptr;
    check(tg_spmm_plan_create(static_cast<int64_t>(a.rows()), static_cast<int64_t>(a.nnz()), rp,
                              max_f, 0, nullptr, &m.plan));
    m.plan_max_f = max_f;
    m.plan_version = a.version();
    return m.plan;
}

void sync() {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) hip_fail(e, "hipDeviceSynchronize");
}

std::string dims(size_t r, size_t c) { return std::to_string(r) + "\xC3\x97" + std::to_string(c); }

}  // namespace detail

using detail::Access;
using detail::check;

// ===========================================================================
// Tensor (tensor.hpp / tensor.cpp:12-174)
// ===========================================================================
Tensor::Tensor() : shape_{0, 0}, strides_{0, 0} {}  // tensor.cpp:12-15

Tensor::~Tensor() = default;

Tensor::Tensor(const Tensor& o)
    : format_(o.format_), shape_(o.shape_), strides_(o.strides_), count_(o.count_) {
    o.sync_host();
    data_ = o.data_;
    row_ptr_ = o.row_ptr_;
    col_ind_ = o.col_ind_;
    host_valid_ = true;
}

Tensor::Tensor(Tensor&& o) noexcept
    : format_(o.format_),
      shape_(std::move(o.shape_)),
      strides_(std::move(o.strides_)),
      count_(o.count_),
      data_(std::move(o.data_)),
      row_ptr_(std::move(o.row_ptr_)),
      col_ind_(std::move(o.col_ind_)),
      host_valid_(o.host_valid_),
      dev_(std::move(o.dev_)),
      version_(o.version_) {
    o.shape_ = {0, 0};
    o.strides_ = {0, 0};
    o.count_ = 0;
    o.host_valid_ = true;
}

Tensor& Tensor::operator=(const Tensor& o) {
    if (this != &o) {
        Tensor t(o);
        *this = std::move(t);
    }
    return *this;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        format_ = o.format_;
        shape_ = std::move(o.shape_);
        strides_ = std::move(o.strides_);
        count_ = o.count_;
        data_ = std::move(o.data_);
        row_ptr_ = std::move(o.row_ptr_);
        col_ind_ = std::move(o.col_ind_);
        host_valid_ = o.host_valid_;
        dev_ = std::move(o.dev_);
        ++version_;
        o.shape_ = {0, 0};
        o.strides_ = {0, 0};
        o.count_ = 0;
        o.host_valid_ = true;
    }
    return *this;
}

Tensor Tensor::dense(std::size_t rows, std::size_t cols) {
    return dense(rows, cols, std::vector<float>(rows * cols, 0.0f));
}

Tensor Tensor::dense(std::size_t rows, std::size_t cols, std::vector<float> data) {
    if (data.size() != rows * cols)
        throw std::invalid_argument("Tensor::dense: data.size() (" + std::to_string(data.size()) +
                                    ") != rows*cols (" + std::to_string(rows * cols) + ")");
    Tensor t;
    t.format_ = StorageFormat::Dense;
    t.shape_ = {rows, cols};
    t.strides_ = {cols, 1};
    t.count_ = rows * cols;
    t.data_ = std::move(data);
    return t;
}

Tensor Tensor::sparse_csr(std::size_t rows, std::size_t cols, std::vector<int32_t> row_ptr,
                          std::vector<int32_t> col_ind, std::vector<float> values) {
    // tensor.cpp:46-86, in the reference's order and wording
    if (row_ptr.size() != rows + 1)
        throw std::invalid_argument("Tensor::sparse_csr: row_ptr.size() (" +
                                    std::to_string(row_ptr.size()) + ") must equal rows+1 (" +
                                    std::to_string(rows + 1) + ")");
    if (col_ind.size() != values.size())
        throw std::invalid_argument("Tensor::sparse_csr: col_ind.size() (" +
                                    std::to_string(col_ind.size()) +
                                    ") must equal values.size() (" +
                                    std::to_string(values.size()) + ")");
    const auto nnz = static_cast<std::size_t>(row_ptr.back());
    if (nnz != values.size())
        throw std::invalid_argument("Tensor::sparse_csr: row_ptr.back() (" + std::to_string(nnz) +
                                    ") must equal values.size() (" +
                                    std::to_string(values.size()) + ")");
    for (std::size_t i = 0; i < col_ind.size(); ++i)
        if (col_ind[i] < 0 || static_cast<std::size_t>(col_ind[i]) >= cols)
            throw std::invalid_argument("Tensor::sparse_csr: col_ind[" + std::to_string(i) +
                                        "] = " + std::to_string(col_ind[i]) +
                                        " is out of bounds for cols=" + std::to_string(cols));
    for (std::size_t i = 1; i < row_ptr.size(); ++i)
        if (row_ptr[i] < row_ptr[i - 1])
            throw std::invalid_argument(
                "Tensor::sparse_csr: row_ptr must be non-decreasing; row_ptr[" +
                std::to_string(i) + "] = " + std::to_string(row_ptr[i]) + " < row_ptr[" +
                std::to_string(i - 1) + "] = " + std::to_string(row_ptr[i - 1]));
    Tensor t;
    t.format_ = StorageFormat::SparseCSR;
    t.shape_ = {rows, cols};
    t.strides_ = {};
    t.count_ = values.size();
    t.row_ptr_ = std::move(row_ptr);
    t.col_ind_ = std::move(col_ind);
    t.data_ = std::move(values);
    return t;
}

std::size_t Tensor::memory_footprint_bytes() const noexcept {
    if (format_ == StorageFormat::Dense) return count_ * sizeof(float);
    return count_ * sizeof(float) + count_ * sizeof(int32_t) + (shape_[0] + 1) * sizeof(int32_t);
}

void Tensor::sync_host() const {
    if (host_valid_) return;
    detail::sync();
    data_.resize(count_);
    detail::d2h(data_.data(), dev_->data.p, count_ * sizeof(float));
    if (format_ == StorageFormat::SparseCSR) {
        row_ptr_.resize(shape_[0] + 1);
        col_ind_.resize(count_);
        detail::d2h(row_ptr_.data(), dev_->rp.p, row_ptr_.size() * sizeof(int32_t));
        detail::d2h(col_ind_.data(), dev_->ci.p, count_ * sizeof(int32_t));
    }
    host_valid_ = true;
}

const std::vector<float>& Tensor::data() const {
    sync_host();
    return data_;
}

std::vector<float>& Tensor::data() {
    sync_host();
    if (dev_) dev_->valid = false;
    ++version_;
    return data_;
}

const std::vector<int32_t>& Tensor::row_ptr() const {
    sync_host();
    return row_ptr_;
}

const std::vector<int32_t>& Tensor::col_ind() const {
    sync_host();
    return col_ind_;
}

float Tensor::at(std::size_t row, std::size_t col) const {
    if (format_ != StorageFormat::Dense)
        throw std::runtime_error("Tensor::at() is only supported for Dense tensors");
    if (row >= shape_[0] || col >= shape_[1])
        throw std::out_of_range("Tensor::at(" + std::to_string(row) + ", " + std::to_string(col) +
                                ") out of range for shape (" + std::to_string(shape_[0]) + ", " +
                                std::to_string(shape_[1]) + ")");
    return data()[row * strides_[0] + col * strides_[1]];
}

float& Tensor::at(std::size_t row, std::size_t col) {
    if (format_ != StorageFormat::Dense)
        throw std::runtime_error("Tensor::at() is only supported for Dense tensors");
    if (row >= shape_[0] || col >= shape_[1])
        throw std::out_of_range("Tensor::at(" + std::to_string(row) + ", " + std::to_string(col) +
                                ") out of range for shape (" + std::to_string(shape_[0]) + ", " +
                                std::to_string(shape_[1]) + ")");
    return data()[row * strides_[0] + col * strides_[1]];
}

std::string Tensor::repr() const {
    std::ostringstream os;
    os << "Tensor(" << shape_[0] << "x" << shape_[1] << ", "
       << (format_ == StorageFormat::Dense ? "Dense" : "SparseCSR") << ", "
       << memory_footprint_bytes() << " bytes)";
    return os.str();
}

detail::DeviceMirror& Tensor::mirror() const {
    if (!dev_) dev_ = std::make_shared<detail::DeviceMirror>();
    if (!dev_->valid) {
        // host is the valid copy: upload everything
        dev_->data.ensure(count_ * sizeof(float));
        detail::h2d(dev_->data.p, data_.data(), count_ * sizeof(float));
        if (format_ == StorageFormat::SparseCSR) {
            dev_->rp.ensure(row_ptr_.size() * sizeof(int32_t));
            dev_->ci.ensure(count_ * sizeof(int32_t));
            detail::h2d(dev_->rp.p, row_ptr_.data(), row_ptr_.size() * sizeof(int32_t));
            detail::h2d(dev_->ci.p, col_ind_.data(), count_ * sizeof(int32_t));
        }
        dev_->valid = true;
    }
    return *dev_;
}

bool Tensor::device_valid() const noexcept { return dev_ && dev_->valid; }

const float* Tensor::device_data() const { return static_cast<const float*>(mirror().data.p); }

float* Tensor::device_data_mutable() {
    float* p = static_cast<float*>(mirror().data.p);
    host_valid_ = false;
    ++version_;
    return p;
}

const int32_t* Tensor::device_row_ptr() const {
    return static_cast<const int32_t*>(mirror().rp.p);
}

const int32_t* Tensor::device_col_ind() const {
    return static_cast<const int32_t*>(mirror().ci.p);
}

void Tensor::mark_device_written() {
    mirror();
    host_valid_ = false;
    ++version_;
}

Tensor Tensor::device_dense(std::size_t rows, std::size_t cols) {
    return Access::make(StorageFormat::Dense, rows, cols, rows * cols);
}

Tensor Tensor::device_csr(std::size_t rows, std::size_t cols, std::size_t nnz) {
    return Access::make(StorageFormat::SparseCSR, rows, cols, nnz);
}

// ===========================================================================
// ops (ops.hpp / ops.cpp)
// ===========================================================================
namespace {

void require_dense(const Tensor& X, const char* fn) {
    // ops.cpp:303-310
    if (X.format() != StorageFormat::Dense)
        throw std::invalid_argument(std::string(fn) +
                                    ": tensor must be Dense (got SparseCSR). "
                                    "Activations operate on dense feature matrices only.");
}

void require_square_csr(const Tensor& A, const char* fn) {
    // layers.cpp:43-53
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument(std::string(fn) + ": A must be SparseCSR (got Dense).");
    if (A.rows() != A.cols())
        throw std::invalid_argument(std::string(fn) + ": A must be square — got (" +
                                    detail::dims(A.rows(), A.cols()) + ").");
}

int64_t i64(std::size_t v) { return static_cast<int64_t>(v); }

}  // namespace

Tensor matmul(const Tensor& A, const Tensor& B) {
    // ops.cpp:72-97
    if (A.format() != StorageFormat::Dense)
        throw std::invalid_argument(
            "matmul: tensor A must be Dense (got SparseCSR). "
            "Sparse-dense matmul is planned for Phase 4 (SpMM kernel).");
    if (B.format() != StorageFormat::Dense)
        throw std::invalid_argument(
            "matmul: tensor B must be Dense (got SparseCSR). "
            "Sparse-dense matmul is planned for Phase 4 (SpMM kernel).");
    if (A.cols() != B.rows())
        throw std::invalid_argument("matmul: dimension mismatch — A is (" +
                                    detail::dims(A.rows(), A.cols()) + ") but B is (" +
                                    detail::dims(B.rows(), B.cols()) +
                                    "). Required: A.cols() == B.rows() (both = " +
                                    std::to_string(A.cols()) + " vs " + std::to_string(B.rows()) +
                                    ").");
    Tensor C = Tensor::device_dense(A.rows(), B.cols());
    if (C.numel() == 0) return Tensor::dense(A.rows(), B.cols());
    check(tg_matmul(i64(A.rows()), i64(A.cols()), i64(B.cols()), A.device_data(),
                    i64(A.cols()), B.device_data(), i64(B.cols()), C.device_data_mutable(),
                    i64(B.cols()), nullptr, TG_EPI_NONE, TG_GEMM_AUTO, nullptr));
    return C;
}

Tensor spmm(const Tensor& A, const Tensor& B) { return spmm(A, B, SpmmOrder::Exact); }

Tensor spmm(const Tensor& A, const Tensor& B, SpmmOrder order) {
    // ops.cpp:200-236
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument(
            "spmm: tensor A must be SparseCSR (got Dense). "
            "For Dense × Dense, use matmul() instead.");
    if (B.format() != StorageFormat::Dense)
        throw std::invalid_argument(
            "spmm: tensor B must be Dense (got SparseCSR). "
            "Sparse × Sparse multiplication is not supported.");
    if (A.cols() != B.rows())
        throw std::invalid_argument("spmm: dimension mismatch — A is (" +
                                    detail::dims(A.rows(), A.cols()) +
                                    ", SparseCSR) but B is (" + detail::dims(B.rows(), B.cols()) +
                                    ", Dense). Required: A.cols() == B.rows() (" +
                                    std::to_string(A.cols()) + " vs " + std::to_string(B.rows()) +
                                    ").");
    if (A.rows() == 0 || B.cols() == 0 || A.nnz() == 0) return Tensor::dense(A.rows(), B.cols());
    Tensor C = Tensor::device_dense(A.rows(), B.cols());
    tg_spmm_plan_t plan = detail::plan_for(A, i64(B.cols()));
    check(tg_spmm_plan_set_precision(
        plan, order == SpmmOrder::Exact ? TG_PRECISION_EXACT : TG_PRECISION_FAST));
    check(tg_spmm_execute(plan, i64(A.cols()), i64(B.cols()), A.device_row_ptr(),
                          A.device_col_ind(), A.device_data(), B.device_data(), i64(B.cols()),
                          C.device_data_mutable(), i64(B.cols()), nullptr));
    return C;
}

void relu_inplace(Tensor& X) {
    require_dense(X, "relu_inplace");
    if (X.numel()) check(tg_relu(i64(X.numel()), X.device_data_mutable(), nullptr));
}
void leaky_relu_inplace(Tensor& X, float alpha) {
    require_dense(X, "leaky_relu_inplace");
    if (X.numel()) check(tg_leaky_relu(i64(X.numel()), X.device_data_mutable(), alpha, nullptr));
}
void elu_inplace(Tensor& X, float alpha) {
    require_dense(X, "elu_inplace");
    if (X.numel()) check(tg_elu(i64(X.numel()), X.device_data_mutable(), alpha, nullptr));
}
void sigmoid_inplace(Tensor& X) {
    require_dense(X, "sigmoid_inplace");
    if (X.numel()) check(tg_sigmoid(i64(X.numel()), X.device_data_mutable(), nullptr));
}
void tanh_inplace(Tensor& X) {
    require_dense(X, "tanh_inplace");
    if (X.numel()) check(tg_tanh(i64(X.numel()), X.device_data_mutable(), nullptr));
}
void gelu_inplace(Tensor& X) {
    require_dense(X, "gelu_inplace");
    if (X.numel()) check(tg_gelu(i64(X.numel()), X.device_data_mutable(), nullptr));
}
void softmax_inplace(Tensor& X) {
    require_dense(X, "softmax_inplace");
    if (X.cols() == 0) check(tg_softmax(i64(X.rows()), 0, nullptr, nullptr));
    if (X.rows() == 0) return;
    check(tg_softmax(i64(X.rows()), i64(X.cols()), X.device_data_mutable(), nullptr));
}
void log_softmax_inplace(Tensor& X) {
    require_dense(X, "log_softmax_inplace");
    if (X.cols() == 0) check(tg_log_softmax(i64(X.rows()), 0, nullptr, nullptr));
    if (X.rows() == 0) return;
    check(tg_log_softmax(i64(X.rows()), i64(X.cols()), X.device_data_mutable(), nullptr));
}
void add_bias(Tensor& X, const Tensor& bias) {
    // ops.cpp:622-640
    require_dense(X, "add_bias (X)");
    if (bias.format() != StorageFormat::Dense)
        throw std::invalid_argument("add_bias: bias tensor must be Dense (got SparseCSR).");
    if (bias.rows() != 1 || bias.cols() != X.cols())
        throw std::invalid_argument("add_bias: bias must be shape (1×" + std::to_string(X.cols()) +
                                    ") to match X columns, but got (" +
                                    detail::dims(bias.rows(), bias.cols()) + ").");
    if (X.numel() == 0) return;
    check(tg_add_bias(i64(X.rows()), i64(X.cols()), X.device_data_mutable(), bias.device_data(),
                      nullptr));
}

// ===========================================================================
// Graph utilities (layers.cpp:71-208, :359-435, :768-822)
// ===========================================================================
namespace {

Tensor self_loops(const Tensor& A, bool norm) {
    const size_t n = A.rows(), nnz = A.nnz();
    Tensor out = Tensor::device_csr(n, n, nnz + n);
    if (norm)
        check(tg_gcn_norm(i64(n), i64(nnz), A.device_row_ptr(), A.device_col_ind(),
                          A.device_data(), Access::rp(out), Access::ci(out), Access::val(out),
                          nullptr, nullptr, nullptr, 0, nullptr));
    else
        check(tg_add_self_loops(i64(n), i64(nnz), A.device_row_ptr(), A.device_col_ind(),
                                A.device_data(), Access::rp(out), Access::ci(out),
                                Access::val(out), nullptr, 0, nullptr));
    int32_t total = 0;
    detail::d2h(&total, Access::rp(out) + n, sizeof(total));
    Access::set_count(out, static_cast<size_t>(total));
    return out;
}

}  // namespace

Tensor add_self_loops(const Tensor& A) {
    require_square_csr(A, "add_self_loops");
    return self_loops(A, false);
}

Tensor gcn_norm(const Tensor& A) {
    require_square_csr(A, "gcn_norm");
    return self_loops(A, true);
}

Tensor edge_softmax(const Tensor& A) {
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument("edge_softmax: input must be SparseCSR (got Dense).");
    Tensor out = Tensor::device_csr(A.rows(), A.cols(), A.nnz());
    detail::d2d(Access::rp(out), A.device_row_ptr(), (A.rows() + 1) * sizeof(int32_t));
    detail::d2d(Access::ci(out), A.device_col_ind(), A.nnz() * sizeof(int32_t));
    if (A.nnz()) {
        hipError_t e = hipMemset(Access::val(out), 0, A.nnz() * sizeof(float));
        if (e != hipSuccess) detail::hip_fail(e, "hipMemset");
    }
    if (A.rows())
        check(tg_edge_softmax(i64(A.rows()), A.device_row_ptr(), A.device_data(),
                              Access::val(out), nullptr));
    return out;
}

Tensor sage_max_aggregate(const Tensor& A, const Tensor& H) {
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument("sage_max_aggregate: A must be SparseCSR (got Dense).");
    if (H.format() != StorageFormat::Dense)
        throw std::invalid_argument("sage_max_aggregate: H must be Dense (got SparseCSR).");
    if (A.cols() != H.rows())
        throw std::invalid_argument("sage_max_aggregate: A.cols() (" + std::to_string(A.cols()) +
                                    ") != H.rows() (" + std::to_string(H.rows()) + ").");
    Tensor out = Tensor::device_dense(A.rows(), H.cols());
    if (out.numel() == 0) return Tensor::dense(A.rows(), H.cols());
    tg_spmm_plan_t plan = detail::plan_for(A, i64(H.cols()));
    check(tg_sage_aggregate(plan, i64(A.rows()), i64(H.cols()), TG_AGG_MAX, A.device_row_ptr(),
                            A.device_col_ind(), H.device_data(), i64(H.cols()),
                            out.device_data_mutable(), i64(H.cols()), nullptr));
    return out;
}

// ===========================================================================
// Layers (layers.cpp:213-1129)
// ===========================================================================
namespace {

void set_checked(Tensor& dst, Tensor w, size_t r, size_t c, const char* what,
                 const char* dense_msg) {
    if (w.format() != StorageFormat::Dense) throw std::invalid_argument(dense_msg);
    if (w.rows() != r || w.cols() != c)
        throw std::invalid_argument(std::string(what) + ": expected shape (" +
                                    detail::dims(r, c) + "), got (" +
                                    detail::dims(w.rows(), w.cols()) + ").");
    dst = std::move(w);
}

void check_features(const char* layer, size_t h_cols, size_t in_f) {
    if (h_cols != in_f)
        throw std::invalid_argument(std::string(layer) + "::forward: H has " +
                                    std::to_string(h_cols) +
                                    " columns but layer expects in_features=" +
                                    std::to_string(in_f) + ".");
}

}  // namespace

GCNLayer::GCNLayer(std::size_t in_features, std::size_t out_features, bool use_bias,
                   Activation act)
    : in_features_(in_features),
      out_features_(out_features),
      use_bias_(use_bias),
      activation_(act),
      weight_(Tensor::dense(in_features, out_features)),
      bias_(Tensor::dense(1, out_features)) {
    if (in_features == 0) throw std::invalid_argument("GCNLayer: in_features must be > 0.");
    if (out_features == 0) throw std::invalid_argument("GCNLayer: out_features must be > 0.");
}

void GCNLayer::set_weight(Tensor w) {
    set_checked(weight_, std::move(w), in_features_, out_features_, "GCNLayer::set_weight",
                "GCNLayer::set_weight: weight must be Dense.");
}

void GCNLayer::set_bias(Tensor b) {
    if (!use_bias_)
        throw std::invalid_argument(
            "GCNLayer::set_bias: layer was constructed with use_bias=false.");
    set_checked(bias_, std::move(b), 1, out_features_, "GCNLayer::set_bias",
                "GCNLayer::set_bias: bias must be Dense.");
}

Tensor GCNLayer::forward(const Tensor& A_norm, const Tensor& H) const {
    // layers.cpp:288-316
    if (A_norm.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument(
            "GCNLayer::forward: A_norm must be SparseCSR (got Dense). "
            "Use gcn_norm() to precompute the normalized adjacency.");
    if (A_norm.rows() != A_norm.cols())
        throw std::invalid_argument("GCNLayer::forward: A_norm must be square — got (" +
                                    detail::dims(A_norm.rows(), A_norm.cols()) + ").");
    if (H.format() != StorageFormat::Dense)
        throw std::invalid_argument("GCNLayer::forward: H must be Dense (got SparseCSR).");
    check_features("GCNLayer", H.cols(), in_features_);
    if (A_norm.rows() != H.rows())
        throw std::invalid_argument("GCNLayer::forward: A_norm has " +
                                    std::to_string(A_norm.rows()) + " rows but H has " +
                                    std::to_string(H.rows()) +
                                    " rows. They must match (N nodes).");
    const Tensor hw = matmul(H, weight_);
    if (A_norm.rows() == 0 || hw.cols() == 0 || A_norm.nnz() == 0) {
        // spmm's zero result (ops.cpp:231-236), then the epilogue
        Tensor out = spmm(A_norm, hw);
        if (use_bias_) add_bias(out, bias_);
        if (activation_ == Activation::ReLU) relu_inplace(out);
        return out;
    }
    // spmm, add_bias and relu_inplace (layers.cpp:319-336) as one pass: the
    // bias and the activation are applied in the SpMM's store, bit-identical
    // to the three calls
    const int64_t f = i64(hw.cols());
    Tensor out = Tensor::device_dense(A_norm.rows(), hw.cols());
    tg_spmm_plan_t plan = detail::plan_for(A_norm, f);
    check(tg_spmm_plan_set_precision(plan, TG_PRECISION_EXACT));
    check(tg_spmm_execute_epilogue(
        plan, i64(A_norm.cols()), f, A_norm.device_row_ptr(), A_norm.device_col_ind(),
        A_norm.device_data(), hw.device_data(), f, out.device_data_mutable(), f,
        use_bias_ ? bias_.device_data() : nullptr,
        activation_ == Activation::ReLU ? TG_EPI_RELU : TG_EPI_NONE, nullptr));
    return out;
}

SAGELayer::SAGELayer(std::size_t in_features, std::size_t out_features, Aggregator agg,
                     bool use_bias, Activation act)
    : in_features_(in_features),
      out_features_(out_features),
      aggregator_(agg),
      use_bias_(use_bias),
      activation_(act),
      weight_neigh_(Tensor::dense(in_features, out_features)),
      weight_self_(Tensor::dense(in_features, out_features)),
      bias_(Tensor::dense(1, out_features)) {
    if (in_features == 0) throw std::invalid_argument("SAGELayer: in_features must be > 0.");
    if (out_features == 0) throw std::invalid_argument("SAGELayer: out_features must be > 0.");
}

void SAGELayer::set_weight_neigh(Tensor w) {
    set_checked(weight_neigh_, std::move(w), in_features_, out_features_,
                "SAGELayer::set_weight_neigh", "SAGELayer::set_weight_neigh: weight must be Dense.");
}

void SAGELayer::set_weight_self(Tensor w) {
    set_checked(weight_self_, std::move(w), in_features_, out_features_,
                "SAGELayer::set_weight_self", "SAGELayer::set_weight_self: weight must be Dense.");
}

void SAGELayer::set_bias(Tensor b) {
    if (!use_bias_)
        throw std::invalid_argument(
            "SAGELayer::set_bias: layer was constructed with use_bias=false.");
    set_checked(bias_, std::move(b), 1, out_features_, "SAGELayer::set_bias",
                "SAGELayer::set_bias: bias must be Dense.");
}

Tensor SAGELayer::forward(const Tensor& A, const Tensor& H) const {
    // layers.cpp:540-560
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument("SAGELayer::forward: A must be SparseCSR (got Dense).");
    if (H.format() != StorageFormat::Dense)
        throw std::invalid_argument("SAGELayer::forward: H must be Dense (got SparseCSR).");
    check_features("SAGELayer", H.cols(), in_features_);
    if (A.cols() != H.rows())
        throw std::invalid_argument("SAGELayer::forward: A.cols() (" + std::to_string(A.cols()) +
                                    ") != H.rows() (" + std::to_string(H.rows()) + ").");
    Tensor out = Tensor::device_dense(A.rows(), out_features_);
    if (A.rows() == 0) return Tensor::dense(0, out_features_);
    const int agg = aggregator_ == Aggregator::Mean ? TG_AGG_MEAN : TG_AGG_MAX;
    tg_spmm_plan_t plan =
        detail::plan_for(A, i64(std::max(in_features_, 2 * out_features_)));
    check(tg_sage_forward(plan, i64(A.rows()), i64(in_features_), i64(out_features_), agg,
                          A.device_row_ptr(), A.device_col_ind(), H.device_data(),
                          weight_neigh_.device_data(), weight_self_.device_data(),
                          use_bias_ ? bias_.device_data() : nullptr,
                          activation_ == Activation::ReLU ? TG_ACT_RELU : TG_ACT_NONE,
                          TG_POST_NONE, TG_SAGE_AUTO, out.device_data_mutable(), nullptr, 0,
                          nullptr));
    return out;
}

GATLayer::GATLayer(std::size_t in_features, std::size_t out_features, float negative_slope,
                   bool use_bias, Activation act)
    : in_features_(in_features),
      out_features_(out_features),
      negative_slope_(negative_slope),
      use_bias_(use_bias),
      activation_(act),
      weight_(Tensor::dense(in_features, out_features)),
      attn_left_(Tensor::dense(1, out_features)),
      attn_right_(Tensor::dense(1, out_features)),
      bias_(Tensor::dense(1, out_features)) {
    if (in_features == 0) throw std::invalid_argument("GATLayer: in_features must be > 0.");
    if (out_features == 0) throw std::invalid_argument("GATLayer: out_features must be > 0.");
}

void GATLayer::set_weight(Tensor w) {
    set_checked(weight_, std::move(w), in_features_, out_features_, "GATLayer::set_weight",
                "GATLayer::set_weight: weight must be Dense.");
}

void GATLayer::set_attn_left(Tensor a) {
    set_checked(attn_left_, std::move(a), 1, out_features_, "GATLayer::set_attn_left",
                "GATLayer::set_attn_left: attention vector must be Dense.");
}

void GATLayer::set_attn_right(Tensor a) {
    set_checked(attn_right_, std::move(a), 1, out_features_, "GATLayer::set_attn_right",
                "GATLayer::set_attn_right: attention vector must be Dense.");
}

void GATLayer::set_bias(Tensor b) {
    if (!use_bias_)
        throw std::invalid_argument(
            "GATLayer::set_bias: layer was constructed with use_bias=false.");
    set_checked(bias_, std::move(b), 1, out_features_, "GATLayer::set_bias",
                "GATLayer::set_bias: bias must be Dense.");
}

Tensor GATLayer::forward(const Tensor& A, const Tensor& H) const {
    // layers.cpp:945-975
    if (A.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument(
            "GATLayer::forward: A must be SparseCSR (got Dense). "
            "Use add_self_loops() to prepare the adjacency.");
    if (A.rows() != A.cols())
        throw std::invalid_argument("GATLayer::forward: A must be square — got (" +
                                    detail::dims(A.rows(), A.cols()) + ").");
    if (H.format() != StorageFormat::Dense)
        throw std::invalid_argument("GATLayer::forward: H must be Dense (got SparseCSR).");
    check_features("GATLayer", H.cols(), in_features_);
    if (A.rows() != H.rows())
        throw std::invalid_argument("GATLayer::forward: A has " + std::to_string(A.rows()) +
                                    " rows but H has " + std::to_string(H.rows()) +
                                    " rows. They must match (N nodes).");
    const size_t n = A.rows(), f = out_features_;
    if (n == 0) return Tensor::dense(0, f);
    Tensor wh = matmul(H, weight_);
    Tensor scores = Tensor::device_dense(2, n);
    float* src = scores.device_data_mutable();
    float* dst = src + n;
    check(tg_gat_scores(i64(n), 1, i64(f), wh.device_data(), i64(f), attn_left_.device_data(),
                        attn_right_.device_data(), src, dst, nullptr));
    Tensor out = Tensor::device_dense(n, f);
    tg_spmm_plan_t plan = detail::plan_for(A, i64(f));
    check(tg_gat_aggregate(plan, i64(n), 1, i64(f), A.device_row_ptr(), A.device_col_ind(),
                           wh.device_data(), i64(f), src, dst, negative_slope_,
                           use_bias_ ? bias_.device_data() : nullptr,
                           activation_ == Activation::ReLU ? TG_ACT_RELU : TG_ACT_NONE,
                           TG_POST_NONE, 1, out.device_data_mutable(), i64(f), nullptr, 0,
                           nullptr));
    return out;  // `scores` and `wh` are released in stream order
}

// ===========================================================================
// Model (model.hpp / model.cpp:191-439) over tg_model_*
// ===========================================================================
struct Model::Impl {
    tg_model_t h = nullptr;
    std::weak_ptr<detail::DeviceMirror> adj;  // the adjacency the cache was built for
    uint64_t adj_version = 0;
    ~Impl() {
        if (h) tg_model_destroy(h);
    }
};

Model::Model() : impl_(new Impl) { check(tg_model_create(&impl_->h)); }
Model::~Model() = default;
Model::Model(Model&&) noexcept = default;
Model& Model::operator=(Model&&) noexcept = default;

namespace {
int post_code(Model::InterActivation p) {
    return p == Model::InterActivation::ReLU ? TG_POST_RELU
           : p == Model::InterActivation::ELU ? TG_POST_ELU
                                              : TG_POST_NONE;
}
int act_code(Activation a) { return a == Activation::ReLU ? TG_ACT_RELU : TG_ACT_NONE; }
}  // namespace

std::size_t Model::add_gcn_layer(std::size_t in_f, std::size_t out_f, bool bias, Activation act,
                                 InterActivation post) {
    int64_t idx = 0;
    check(tg_model_add_gcn_layer(impl_->h, i64(in_f), i64(out_f), bias, act_code(act),
                                 post_code(post), &idx));
    num_layers_ = static_cast<size_t>(idx) + 1;
    return static_cast<size_t>(idx);
}

std::size_t Model::add_sage_layer(std::size_t in_f, std::size_t out_f, SAGELayer::Aggregator agg,
                                  bool bias, Activation act, InterActivation post) {
    int64_t idx = 0;
    check(tg_model_add_sage_layer(impl_->h, i64(in_f), i64(out_f),
                                  agg == SAGELayer::Aggregator::Mean ? TG_AGG_MEAN : TG_AGG_MAX,
                                  bias, act_code(act), post_code(post), &idx));
    num_layers_ = static_cast<size_t>(idx) + 1;
    return static_cast<size_t>(idx);
}

std::size_t Model::add_gat_layer(std::size_t in_f, std::size_t out_f, std::size_t num_heads,
                                 bool concat, float neg_slope, bool bias, Activation act,
                                 InterActivation post) {
    int64_t idx = 0;
    check(tg_model_add_gat_layer(impl_->h, i64(in_f), i64(out_f), i64(num_heads), concat,
                                 neg_slope, bias, act_code(act), post_code(post), &idx));
    num_layers_ = static_cast<size_t>(idx) + 1;
    return static_cast<size_t>(idx);
}

void Model::load_weights(const WeightFile& wf) {
    check(tg_model_clear_tensors(impl_->h));
    for (const auto& kv : wf.tensors) {
        const Tensor& t = kv.second;
        if (t.format() != StorageFormat::Dense)
            throw std::invalid_argument("Model::load_weights: tensor '" + kv.first +
                                        "' must be Dense.");
        check(tg_model_set_tensor(impl_->h, kv.first.c_str(), i64(t.rows()), i64(t.cols()),
                                  t.data().data()));
    }
    check(tg_model_load_weights(impl_->h));
}

Tensor Model::forward(const Tensor& adjacency, const Tensor& features) const {
    if (num_layers_ == 0) throw std::runtime_error("Model::forward: no layers configured.");
    if (adjacency.format() != StorageFormat::SparseCSR)
        throw std::invalid_argument("Model::forward: adjacency must be SparseCSR (got Dense).");
    if (features.format() != StorageFormat::Dense)
        throw std::invalid_argument("Model::forward: features must be Dense (got SparseCSR).");
    if (adjacency.rows() != adjacency.cols())
        throw std::invalid_argument("Model::forward: adjacency must be square — got (" +
                                    detail::dims(adjacency.rows(), adjacency.cols()) + ").");
    if (adjacency.rows() != features.rows())
        throw std::invalid_argument("Model::forward: adjacency has " +
                                    std::to_string(adjacency.rows()) + " rows but features has " +
                                    std::to_string(features.rows()) + " rows.");
    int64_t cols = 0;
    check(tg_model_output_cols(impl_->h, &cols));
    const size_t n = adjacency.rows();
    const int32_t* rp = adjacency.device_row_ptr();
    // Reuse the derived adjacency only for the same, unedited tensor (the
    // same device copy, which no other tensor shares, at the same version).
    std::shared_ptr<detail::DeviceMirror> mp = Access::mirror_ptr(adjacency);
    const bool same = impl_->adj.lock() == mp && impl_->adj_version == adjacency.version();
    Tensor out = Tensor::device_dense(n, static_cast<size_t>(cols));
    check(tg_model_forward(impl_->h, i64(n), i64(adjacency.nnz()), rp,
                           adjacency.device_col_ind(), adjacency.device_data(),
                           i64(features.cols()), features.device_data(),
                           n ? out.device_data_mutable() : nullptr,
                           same ? TG_FORWARD_CACHED : TG_FORWARD_REFERENCE, nullptr));
    impl_->adj = mp;
    impl_->adj_version = adjacency.version();
    return out;
}

// ===========================================================================
// GraphLoader::edge_list_to_csr (graph_loader.cpp:211-281)
// ===========================================================================
Tensor GraphLoader::edge_list_to_csr(const std::vector<std::pair<int32_t, int32_t>>& edges,
                                     std::size_t num_nodes) {
    const size_t e = edges.size();
    if (num_nodes == 0 && e != 0)  // graph_loader.cpp:216-221, before any device work
        throw std::invalid_argument(
            "GraphLoader::edge_list_to_csr: num_nodes is 0 but edges is non-empty");
    std::vector<int32_t> src(e), dst(e);
    for (size_t i = 0; i < e; ++i) {
        src[i] = edges[i].first;
        dst[i] = edges[i].second;
    }
    Tensor ends = Tensor::device_dense(2, e);
    int32_t* d_src = reinterpret_cast<int32_t*>(ends.device_data_mutable());
    int32_t* d_dst = d_src + e;
    detail::h2d(d_src, src.data(), e * sizeof(int32_t));
    detail::h2d(d_dst, dst.data(), e * sizeof(int32_t));
    Tensor out = Tensor::device_csr(num_nodes, num_nodes, e);
    check(tg_edge_list_to_csr(i64(num_nodes), i64(e), d_src, d_dst, Access::rp(out),
                              Access::ci(out), Access::val(out), nullptr, 0, nullptr));
    return out;
}

}  // namespace tinygnn

// ===========================================================================
// Ingestion: GraphLoader (graph_loader.cpp:61-326), load_weight_file
// (model.cpp:134-185), load_cora_binary (model.cpp:49-129)
// ===========================================================================
namespace tinygnn {
namespace {

struct CsvHandle {
    tg_csv_t h = nullptr;
    explicit CsvHandle(const std::string& path) { check(tg_csv_open(path.c_str(), &h, nullptr)); }
    ~CsvHandle() {
        if (h) tg_csv_destroy(h);
    }
    CsvHandle(const CsvHandle&) = delete;
    CsvHandle& operator=(const CsvHandle&) = delete;
    int64_t n_data() const {
        int64_t n = 0;
        int hdr = 0;
        check(tg_csv_info(h, &n, &hdr));
        return n > hdr ? n - hdr : 0;
    }
};

// Edge endpoints parsed on the device: a 2 x n int32 scratch tensor
// (row 0 = src, row 1 = dst) and the largest endpoint.
Tensor device_edges(const CsvHandle& c, int64_t* max_id) {
    const int64_t n = c.n_data();
    Tensor ends = Tensor::device_dense(2, static_cast<size_t>(n));
    int32_t* d = reinterpret_cast<int32_t*>(ends.device_data_mutable());
    check(tg_csv_parse_edges(c.h, d, d + n, max_id, nullptr));
    return ends;
}

}  // namespace

std::vector<std::pair<int32_t, int32_t>> GraphLoader::parse_edges(const std::string& path) {
    CsvHandle c(path);
    int64_t max_id = -1;
    Tensor ends = device_edges(c, &max_id);
    const size_t n = ends.cols();
    std::vector<int32_t> buf(2 * n);
    detail::d2h(buf.data(), ends.device_data(), 2 * n * sizeof(int32_t));
    std::vector<std::pair<int32_t, int32_t>> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = {buf[i], buf[n + i]};
    return out;
}

Tensor GraphLoader::parse_features(const std::string& path) {
    CsvHandle c(path);
    int64_t rows = 0, cols = 0;
    check(tg_csv_feature_shape(c.h, &rows, &cols, nullptr));
    Tensor out = Tensor::device_dense(static_cast<size_t>(rows), static_cast<size_t>(cols));
    check(tg_csv_parse_features(c.h, rows * cols ? out.device_data_mutable() : nullptr, rows,
                                cols, nullptr));
    return out;
}

GraphData GraphLoader::load(const std::string& edges_path, const std::string& features_path) {
    int64_t max_id = -1;
    CsvHandle ce(edges_path);
    Tensor ends = device_edges(ce, &max_id);
    const int64_t n_edges = static_cast<int64_t>(ends.cols());
    CsvHandle cf(features_path);
    int64_t rows = 0, cols = 0;
    check(tg_csv_feature_shape(cf.h, &rows, &cols, nullptr));
    const int64_t num_nodes = std::max<int64_t>(n_edges ? max_id + 1 : 0, rows);
    GraphData gd;
    gd.node_features = Tensor::device_dense(static_cast<size_t>(num_nodes), static_cast<size_t>(cols));
    check(tg_csv_parse_features(cf.h,
                                num_nodes * cols ? gd.node_features.device_data_mutable() : nullptr,
                                num_nodes, cols, nullptr));
    gd.adjacency = Tensor::device_csr(static_cast<size_t>(num_nodes), static_cast<size_t>(num_nodes),
                                      static_cast<size_t>(n_edges));
    const int32_t* d = reinterpret_cast<const int32_t*>(ends.device_data());
    check(tg_edge_list_to_csr(num_nodes, n_edges, d, d + n_edges, Access::rp(gd.adjacency),
                              Access::ci(gd.adjacency), Access::val(gd.adjacency), nullptr, 0,
                              nullptr));
    gd.num_nodes = static_cast<size_t>(num_nodes);
    gd.num_edges = static_cast<size_t>(n_edges);
    gd.num_features = static_cast<size_t>(cols);
    return gd;
}

WeightFile load_weight_file(const std::string& path) {
    tg_weights_t w = nullptr;
    check(tg_weights_open(path.c_str(), &w));
    struct Close {
        tg_weights_t w;
        ~Close() { tg_weights_destroy(w); }
    } close{w};
    int64_t n = 0;
    WeightFile wf;
    check(tg_weights_info(w, &n, &wf.test_accuracy));
    for (int64_t i = 0; i < n; ++i) {
        const char* name = nullptr;
        const float* data = nullptr;
        int64_t len = 0, rows = 0, cols = 0;
        check(tg_weights_tensor(w, i, &name, &len, &rows, &cols, &data));
        wf.tensors[std::string(name, static_cast<size_t>(len))] = Tensor::dense(
            static_cast<size_t>(rows), static_cast<size_t>(cols),
            std::vector<float>(data, data + rows * cols));
    }
    return wf;
}

void Model::load_weights(const std::string& path) { load_weights(load_weight_file(path)); }

CoraData load_cora_binary(const std::string& path) {
    tg_cora_t c = nullptr;
    check(tg_cora_open(path.c_str(), &c));
    struct Close {
        tg_cora_t c;
        ~Close() { tg_cora_destroy(c); }
    } close{c};
    int64_t n = 0, f = 0, k = 0, e = 0;
    check(tg_cora_info(c, &n, &f, &k, &e));
    CoraData cd;
    cd.num_nodes = static_cast<size_t>(n);
    cd.num_features = static_cast<size_t>(f);
    cd.num_classes = static_cast<size_t>(k);
    cd.num_edges = static_cast<size_t>(e);
    cd.features = Tensor::device_dense(cd.num_nodes, cd.num_features);
    cd.adjacency = Tensor::device_csr(cd.num_nodes, cd.num_nodes, cd.num_edges);
    check(tg_cora_upload(c, n * f ? cd.features.device_data_mutable() : nullptr,
                         Access::rp(cd.adjacency), Access::ci(cd.adjacency),
                         Access::val(cd.adjacency), nullptr));
    const int32_t* labels = nullptr;
    const uint8_t *tr = nullptr, *va = nullptr, *te = nullptr;
    check(tg_cora_host(c, &labels, &tr, &va, &te));
    cd.labels.assign(labels, labels + n);
    cd.train_mask.assign(tr, tr + n);
    cd.val_mask.assign(va, va + n);
    cd.test_mask.assign(te, te + n);
    return cd;
}

}  // namespace tinygnn

namespace tinygnn {

Tensor Tensor::dense_from_device(std::size_t rows, std::size_t cols, const float* device_ptr) {
    Tensor t = device_dense(rows, cols);
    if (rows * cols)
        detail::d2d(t.device_data_mutable(), device_ptr, rows * cols * sizeof(float));
    return t;
}

Tensor csr_from_edge_index(const int32_t* src, const int32_t* dst, std::size_t num_edges,
                           std::size_t num_nodes) {
    Tensor ends = Tensor::device_dense(2, num_edges);
    int32_t* d_src = reinterpret_cast<int32_t*>(ends.device_data_mutable());
    int32_t* d_dst = d_src + num_edges;
    detail::h2d(d_src, src, num_edges * sizeof(int32_t));
    detail::h2d(d_dst, dst, num_edges * sizeof(int32_t));
    Tensor out = Tensor::device_csr(num_nodes, num_nodes, num_edges);
    check(tg_coo_to_csr(static_cast<int64_t>(num_nodes), static_cast<int64_t>(num_edges), d_src,
                        d_dst, Access::rp(out), Access::ci(out), Access::val(out),
                        "from_edge_index", nullptr));
    return out;
}

}  // namespace tinygnn
