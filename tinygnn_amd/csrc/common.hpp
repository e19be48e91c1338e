// common.hpp -- shared plumbing for the gfx950 kernels and the C-ABI layer.
//
// Status convention of the C-ABI (declared in include/tinygnn_amd.h):
// every entry point returns an int status and never lets a C++ exception
// cross the boundary.  TG_ERR_INVALID_ARGUMENT / TG_ERR_RUNTIME /
// TG_ERR_OUT_OF_RANGE name the std:: exception the reference throws in the
// same situation; the message (thread-local) carries the reference's text.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "tinygnn_amd.h"

namespace tg {

// Exceptions used inside the library; converted to status codes at the ABI.
struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct AllocError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_last_error(const std::string& msg);
const char* last_error();

// Runs fn, mapping exceptions to TG_* status codes and the thread-local
// message.  Used by every extern "C" entry point.
template <typename F>
int guard(F&& fn) noexcept {
    try {
        fn();
        return TG_OK;
    } catch (const std::invalid_argument& e) {
        set_last_error(e.what());
        return TG_ERR_INVALID_ARGUMENT;
    } catch (const std::out_of_range& e) {
        set_last_error(e.what());
        return TG_ERR_OUT_OF_RANGE;
    } catch (const HipError& e) {
        set_last_error(e.what());
        return TG_ERR_HIP;
    } catch (const AllocError& e) {
        set_last_error(e.what());
        return TG_ERR_ALLOC;
    } catch (const std::runtime_error& e) {
        set_last_error(e.what());
        return TG_ERR_RUNTIME;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return TG_ERR_RUNTIME;
    } catch (...) {
        set_last_error("unknown error");
        return TG_ERR_RUNTIME;
    }
}

[[noreturn]] void throw_hip(hipError_t e, const char* what, const char* file, int line);

#define TG_HIP(call)                                                      \
    do {                                                                  \
        hipError_t tg_e_ = (call);                                        \
        if (tg_e_ != hipSuccess) ::tg::throw_hip(tg_e_, #call, __FILE__, __LINE__); \
    } while (0)

// Checks the launch status of the kernel just enqueued.
#define TG_LAUNCH_CHECK() TG_HIP(hipGetLastError())

inline void require(bool ok, const std::string& msg) {
    if (!ok) throw std::invalid_argument(msg);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workspace carving: hands out 256-byte aligned slices of a caller buffer.
struct Carver {
    char* base;
    size_t cap;
    size_t used = 0;
    Carver(void* p, size_t c) : base(static_cast<char*>(p)), cap(c) {}
    template <typename T>
    T* take(size_t count) {
        size_t off = (used + 255) & ~size_t(255);
        size_t bytes = count * sizeof(T);
        if (base != nullptr && off + bytes > cap)
            throw std::invalid_argument("workspace too small: need at least " +
                                        std::to_string(off + bytes) + " bytes, got " +
                                        std::to_string(cap));
        used = off + bytes;
        return base ? reinterpret_cast<T*>(base + off) : nullptr;
    }
    size_t bytes() const { return (used + 255) & ~size_t(255); }
};

// RAII device allocation (used by plans and the C++ host API, never by the
// kernels themselves).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { resize(bytes); }
    ~DeviceBuffer() { reset(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) { reset(); p_ = o.p_; n_ = o.n_; o.p_ = nullptr; o.n_ = 0; }
        return *this;
    }
    void resize(size_t bytes);        // discards contents
    void reserve(size_t bytes) { if (bytes > n_) resize(bytes); }
    void reset();
    void* get() const { return p_; }
    template <typename T> T* as() const { return static_cast<T*>(p_); }
    size_t size() const { return n_; }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// RAII pinned host allocation (hipHostMalloc): small device-to-host results
// that the host reads after a stream synchronisation, so that the copies
// themselves stay asynchronous.
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    ~PinnedBuffer() { reset(); }
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    void reserve(size_t bytes);
    void reset();
    template <typename T> T* as() const { return static_cast<T*>(p_); }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// Small fill kernels (used instead of hipMemset*Async so that library calls
// can be captured into HIP graphs).
void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s);
void fill_zero_2d(float* p, int64_t rows, int64_t cols, int64_t ld, hipStream_t s);

// Device exclusive scan of int32 counts: out[i] = sum(in[0..i)), out[n] =
// total (out has n+1 entries).  temp must hold scan_temp_elems(n) int64.
size_t scan_temp_elems(int64_t n);
void exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, int64_t* temp,
                        hipStream_t s);

}  // namespace tg
