// noalloc.hip -- tg_spmm_noalloc: SpMM that allocates nothing.  No
// counterpart in the reference: it is for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The plan lives in one fixed device array per GPU.  It is the only thing in
// this file, which holds no kernel (the kernels are spmm.hip's and take the
// array's address as an argument), so its code object -- and with it the
// array -- is loaded onto a GPU only when a process first resolves the
// array's address there: processes that never call tg_spmm_noalloc do not
// hold it.
#include "common.hpp"
#include "spmm_plan.hpp"

#include <mutex>
#include <string>

// Each GPU holds its own copy from the first tg_spmm_noalloc call on it
// until the process ends; every call on one GPU shares it (overlapping calls
// race).
static __device__ __align__(256) unsigned char scratch[TG_SPMM_NOALLOC_SCRATCH_BYTES];

namespace tg {
namespace {

constexpr int kMaxDevices = 64;

// The array's device address on the current device.  The array's name in
// host code is a host-side stand-in, not a device address, so every use
// goes through the address hipGetSymbolAddress returns, taken once per
// device with that device current.  That first resolution may load the
// code object (an allocation), so it must not happen under stream capture:
// the first call on each device is refused while `s` is capturing.
char* noalloc_scratch(hipStream_t s) {
    int dev = 0;
    TG_HIP(hipGetDevice(&dev));
    require(dev >= 0 && dev < kMaxDevices, "tg_spmm_noalloc: device ordinal out of range");
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        TG_HIP(hipStreamIsCapturing(s, &st));
        require(st == hipStreamCaptureStatusNone,
                "tg_spmm_noalloc: the first call on a device must be made outside stream "
                "capture (it resolves the device array's address); call it once before "
                "capturing");
        void* p = nullptr;
        TG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        require(p != nullptr, "tg_spmm_noalloc: no device address for the scratch array");
        addr[dev] = p;
    }
    return static_cast<char*>(addr[dev]);
}

}  // namespace
}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_spmm_noalloc(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
                    const int32_t* col_ind, const float* val, const float* b, int64_t ldb,
                    float* c, int64_t ldc, tg_stream_t stream) {
    return guard([&] {
        require(m >= 0 && k >= 0 && f >= 0 && nnz >= 0, "spmm: negative dimension");
        require(m < (int64_t(1) << 31) && nnz < (int64_t(1) << 31),
                "spmm: m and nnz must be < 2^31 (int32 CSR)");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (m == 0 || f == 0) return;
        if (nnz == 0) {
            // ops.cpp:231-236: the result is the zero-initialised C.
            tg::fill_zero_2d(c, m, f, ldc, s);
            return;
        }
        require(row_ptr && col_ind && val && b && c, "spmm: null pointer");
        // sizes first: a rejected call does no device work
        const size_t need = tg::spmm_noalloc_bytes(m, nnz, f);
        if (need > TG_SPMM_NOALLOC_SCRATCH_BYTES)
            throw std::invalid_argument(
                "tg_spmm_noalloc: the plan for m=" + std::to_string(m) + ", nnz=" +
                std::to_string(nnz) + ", f=" + std::to_string(f) + " needs " +
                std::to_string(need) + " bytes of scratch; the maximum is " +
                std::to_string(static_cast<size_t>(TG_SPMM_NOALLOC_SCRATCH_BYTES)) +
                " (use tg_spmm or a plan)");
        tg::spmm_noalloc(tg::noalloc_scratch(s), TG_SPMM_NOALLOC_SCRATCH_BYTES, m, f, nnz,
                         row_ptr, col_ind, val, b, ldb, c, ldc, s);
    });
}

}  // extern "C"
