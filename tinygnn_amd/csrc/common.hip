// common.hip -- error plumbing, device buffers and the device-wide scan.
#include "common.hpp"
#include "device_utils.hpp"

#include <string>

namespace tg {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

void throw_hip(hipError_t e, const char* what, const char* file, int line) {
    std::string msg = std::string("HIP error ") + hipGetErrorName(e) + " (" +
                      hipGetErrorString(e) + ") in " + what + " at " + file + ":" +
                      std::to_string(line);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw AllocError(msg);
    throw HipError(msg);
}

void DeviceBuffer::resize(size_t bytes) {
    reset();
    if (bytes == 0) return;
    hipError_t e = hipMalloc(&p_, bytes);
    if (e != hipSuccess) {
        p_ = nullptr;
        (void)hipGetLastError();
        throw AllocError("hipMalloc of " + std::to_string(bytes) + " bytes failed: " +
                         hipGetErrorString(e));
    }
    n_ = bytes;
}

void DeviceBuffer::reset() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = 0;
}

void PinnedBuffer::reserve(size_t bytes) {
    if (bytes <= n_) return;
    reset();
    hipError_t e = hipHostMalloc(&p_, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        p_ = nullptr;
        (void)hipGetLastError();
        throw AllocError("hipHostMalloc of " + std::to_string(bytes) + " bytes failed: " +
                         hipGetErrorString(e));
    }
    n_ = bytes;
}

void PinnedBuffer::reset() {
    if (p_) (void)hipHostFree(p_);
    p_ = nullptr;
    n_ = 0;
}

// ---------------------------------------------------------------------------
// Exclusive scan of int32 counts (tiles of 1024 = 256 threads x 4 items).
// ---------------------------------------------------------------------------
namespace {

constexpr int kScanBlock = 256;
constexpr int kScanItems = 4;
constexpr int kScanTile = kScanBlock * kScanItems;

__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(const int32_t* __restrict__ in,
                                                                 int64_t n,
                                                                 int64_t* __restrict__ part) {
    __shared__ int64_t lds[kScanBlock / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        int64_t i = base + static_cast<int64_t>(j) * kScanBlock + threadIdx.x;
        if (i < n) s += in[i];
    }
    s = wave_sum(s);
    if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t t = 0;
        for (int w = 0; w < kScanBlock / kWave; ++w) t += lds[w];
        part[blockIdx.x] = t;
    }
}

// Single workgroup: exclusive scan of part[0..nb) in place, part[nb] = total.
// 256 threads (one wavefront per SIMD): the workgroup fits beside three
// workgroups of the MFMA GEMM on a compute unit, where a 1,024-thread one
// (62 registers x 4 wavefronts per SIMD) waited for the GEMM's last
// workgroups (0.5 ms in a reference-semantics forward, its plans' scans
// beside layer 0's transform).
__global__ __launch_bounds__(kScanBlock) void scan_parts_kernel(int64_t* __restrict__ part,
                                                                int64_t nb) {
    __shared__ int64_t lds[kScanBlock / kWave];
    int64_t carry = 0;
    for (int64_t base = 0; base < nb; base += kScanBlock) {
        int64_t i = base + threadIdx.x;
        int64_t v = (i < nb) ? part[i] : 0;
        int64_t tot;
        int64_t ex = block_exclusive_scan<kScanBlock>(v, lds, &tot);
        if (i < nb) part[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) part[nb] = carry;
}

__global__ __launch_bounds__(kScanBlock) void scan_apply_kernel(const int32_t* __restrict__ in,
                                                                int32_t* __restrict__ out,
                                                                int64_t n,
                                                                const int64_t* __restrict__ part,
                                                                int64_t nb) {
    __shared__ int64_t lds[kScanBlock / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                         static_cast<int64_t>(threadIdx.x) * kScanItems;
    int64_t v[kScanItems];
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        int64_t i = base + j;
        v[j] = (i < n) ? in[i] : 0;
        s += v[j];
    }
    int64_t tot;
    int64_t ex = block_exclusive_scan<kScanBlock>(s, lds, &tot) + part[blockIdx.x];
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        int64_t i = base + j;
        if (i < n) out[i] = static_cast<int32_t>(ex);
        ex += v[j];
    }
    if (blockIdx.x == nb - 1 && threadIdx.x == 0) out[n] = static_cast<int32_t>(part[nb]);
}

__global__ void scan_empty_kernel(int32_t* out) { out[0] = 0; }

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n,
                                                       int32_t v) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        p[i] = v;
}

__global__ __launch_bounds__(256) void fill_zero_2d_kernel(float* __restrict__ p, int64_t rows,
                                                           int64_t cols, int64_t ld) {
    const int64_t n = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        p[(i / cols) * ld + (i % cols)] = 0.0f;
}

unsigned fill_grid(int64_t n) {
    int64_t b = ceil_div(n, 256);
    return static_cast<unsigned>(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s) {
    if (n <= 0) return;
    fill_i32_kernel<<<fill_grid(n), 256, 0, s>>>(p, n, v);
    TG_LAUNCH_CHECK();
}

void fill_zero_2d(float* p, int64_t rows, int64_t cols, int64_t ld, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    fill_zero_2d_kernel<<<fill_grid(rows * cols), 256, 0, s>>>(p, rows, cols, ld);
    TG_LAUNCH_CHECK();
}

size_t scan_temp_elems(int64_t n) { return static_cast<size_t>(ceil_div(n, kScanTile) + 1); }

void exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, int64_t* temp,
                        hipStream_t s) {
    if (n <= 0) {
        scan_empty_kernel<<<1, 1, 0, s>>>(out);
        TG_LAUNCH_CHECK();
        return;
    }
    const int64_t nb = ceil_div(n, kScanTile);
    scan_reduce_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, s>>>(in, n, temp);
    TG_LAUNCH_CHECK();
    scan_parts_kernel<<<1, kScanBlock, 0, s>>>(temp, nb);
    TG_LAUNCH_CHECK();
    scan_apply_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, s>>>(in, out, n, temp, nb);
    TG_LAUNCH_CHECK();
}

}  // namespace tg

extern "C" {

const char* tg_last_error(void) { return tg::last_error(); }

int tg_version(void) { return (0 << 16) | 1; }

}  // extern "C"
