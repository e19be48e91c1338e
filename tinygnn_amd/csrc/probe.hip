// probe.hip -- a measurement kernel with no counterpart in the reference:
// the L2 read ceiling that the column-blocked aggregation passes, whose
// gathers are L2 hits, are measured against.
//
// Every workgroup streams the whole of one small buffer (a power of two of
// at most a few MB, so each XCD's 4 MB L2 keeps it after the first touch)
// with coalesced 16-byte loads, eight in flight per thread, starting at a
// rotated offset so that the workgroups resident at a time spread over the
// L2 channels.  Nothing but the loads and a running sum is done; one float
// per thread is stored at the end.  Bytes read = workgroups x buffer bytes.
#include "common.hpp"

namespace tg {
namespace {

__global__ __launch_bounds__(256) void l2_read_kernel(const float4* __restrict__ buf,
                                                      int64_t n_vec, float* __restrict__ sink) {
    constexpr int kInFlight = 8;
    const int64_t mask = n_vec - 1;
    // a different start per workgroup (a multiple of the 4 KB a step covers)
    const int64_t rot = (static_cast<int64_t>(blockIdx.x) * 37 * 256 * kInFlight) & mask;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int64_t base = 0; base < n_vec; base += 256 * kInFlight) {
        float4 v[kInFlight];
#pragma unroll
        for (int k = 0; k < kInFlight; ++k)
            v[k] = buf[(base + rot + k * 256 + threadIdx.x) & mask];
#pragma unroll
        for (int k = 0; k < kInFlight; ++k) {
            acc.x += v[k].x;
            acc.y += v[k].y;
            acc.z += v[k].z;
            acc.w += v[k].w;
        }
    }
    sink[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = acc.x + acc.y + acc.z + acc.w;
}

}  // namespace
}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_probe_l2_read(const void* buf, int64_t bytes, int64_t workgroups, float* sink,
                     tg_stream_t stream) {
    return guard([&] {
        require(buf != nullptr && sink != nullptr, "tg_probe_l2_read: null pointer");
        require(bytes >= (int64_t(1) << 15) && (bytes & (bytes - 1)) == 0,
                "tg_probe_l2_read: bytes must be a power of two of at least 32 KB");
        require(reinterpret_cast<uintptr_t>(buf) % 16 == 0,
                "tg_probe_l2_read: buf must be 16-byte aligned");
        require(workgroups >= 1 && workgroups <= (int64_t(1) << 20),
                "tg_probe_l2_read: workgroups must be in [1, 2^20]");
        tg::l2_read_kernel<<<static_cast<unsigned>(workgroups), 256, 0,
                             static_cast<hipStream_t>(stream)>>>(
            static_cast<const float4*>(buf), bytes / 16, sink);
        TG_LAUNCH_CHECK();
    });
}

}  // extern "C"
