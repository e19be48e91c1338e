// tinygnn/tensor.hpp -- the hybrid Dense / CSR tensor of TinyGNN's API
// (reference include/tinygnn/tensor.hpp:14-93), with a device mirror.
//
// The public surface is the reference's: the StorageFormat enum, the
// dense / sparse_csr factories (with their validation and messages), the
// observers, host views through std::vector, at() and repr().  What this
// build adds is residency: a tensor can live in HBM.  Host views are made
// coherent lazily -- a const host accessor copies device data back when the
// device copy is newer; a mutable host accessor (data(), at()) also marks
// the device copy stale, so the next device use uploads the edit.  Device
// accessors upload when the host copy is newer.  Results of device ops are
// device-resident until read.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace tinygnn {

enum class StorageFormat : uint8_t {
    Dense = 0,
    SparseCSR = 1
};

namespace detail {
struct DeviceMirror;  // HBM copies of data / row_ptr / col_ind (+ row plan)
struct Access;        // the library's own ops
}

struct Tensor {
    Tensor();
    Tensor(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(const Tensor& other);
    Tensor& operator=(Tensor&& other) noexcept;
    ~Tensor();

    /// Zero-filled dense rows x cols.
    static Tensor dense(std::size_t rows, std::size_t cols);
    /// Dense rows x cols from row-major data (size must be rows*cols).
    static Tensor dense(std::size_t rows, std::size_t cols, std::vector<float> data);
    /// CSR rows x cols; validated as the reference does (tensor.cpp:41-96).
    static Tensor sparse_csr(std::size_t rows, std::size_t cols, std::vector<int32_t> row_ptr,
                             std::vector<int32_t> col_ind, std::vector<float> values);

    StorageFormat format() const noexcept { return format_; }
    std::size_t rows() const noexcept { return shape_[0]; }
    std::size_t cols() const noexcept { return shape_[1]; }
    std::size_t numel() const noexcept { return count_; }
    std::size_t ndim() const noexcept { return shape_.size(); }
    std::size_t nnz() const noexcept { return count_; }
    std::size_t memory_footprint_bytes() const noexcept;

    const std::vector<std::size_t>& shape() const noexcept { return shape_; }
    const std::vector<std::size_t>& strides() const noexcept { return strides_; }

    // Host views (coherent on access).
    const std::vector<float>& data() const;
    std::vector<float>& data();
    const std::vector<int32_t>& row_ptr() const;
    const std::vector<int32_t>& col_ind() const;

    float at(std::size_t row, std::size_t col) const;
    float& at(std::size_t row, std::size_t col);

    std::string repr() const;

    // ---- device residency (this build's addition) ----------------------
    const float* device_data() const;     // uploads if needed
    float* device_data_mutable();         // uploads if needed; host becomes stale
    const int32_t* device_row_ptr() const;
    const int32_t* device_col_ind() const;
    bool host_valid() const noexcept { return host_valid_; }
    bool device_valid() const noexcept;
    /// Bumped on every mutable access; lets caches notice in-place edits.
    uint64_t version() const noexcept { return version_; }
    /// A tensor whose data lives only in HBM (library results).  For CSR,
    /// `nnz` entries; the device buffers are allocated, contents undefined.
    static Tensor device_dense(std::size_t rows, std::size_t cols);
    /// A dense device-resident copy of rows x cols row-major floats that are
    /// already in device memory (zero-copy interop with other device code).
    static Tensor dense_from_device(std::size_t rows, std::size_t cols, const float* device_ptr);
    static Tensor device_csr(std::size_t rows, std::size_t cols, std::size_t nnz);
    detail::DeviceMirror& mirror() const;  // for the library's own ops
    void mark_device_written();            // device holds the only valid copy

private:
    friend struct detail::Access;
    void sync_host() const;

    StorageFormat format_ = StorageFormat::Dense;
    std::vector<std::size_t> shape_;
    std::vector<std::size_t> strides_;
    std::size_t count_ = 0;  // data elements (Dense: rows*cols, CSR: nnz)
    mutable std::vector<float> data_;
    mutable std::vector<int32_t> row_ptr_;
    mutable std::vector<int32_t> col_ind_;
    mutable bool host_valid_ = true;
    mutable std::shared_ptr<detail::DeviceMirror> dev_;
    uint64_t version_ = 0;
};

}  // namespace tinygnn
