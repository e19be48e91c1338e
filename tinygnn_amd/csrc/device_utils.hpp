// device_utils.hpp -- wave64 / workgroup primitives for gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tg {

constexpr int kWave = 64;  // CDNA wavefront width

// exp evaluated in double and rounded once: the correctly rounded float
// exp except when the double result falls within an ulp of a float
// midpoint; the host libm's expf is within 0.502 ulp, so the two agree but
// for rare last-ulp cases.
__device__ __forceinline__ float exp_rn(float x) {
    return static_cast<float>(exp(static_cast<double>(x)));
}

// Inclusive scan across the 64 lanes of a wavefront.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        T t = __shfl_up(v, d, kWave);
        if (lane >= d) v += t;
    }
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        float o = __shfl_xor(v, d, kWave);
        v = (v < o) ? o : v;
    }
    return v;
}

// Exclusive scan over a workgroup of BLOCK threads (BLOCK multiple of 64).
// Returns the exclusive prefix of v and writes the workgroup total to *total.
// `lds` must hold BLOCK/64 elements.  Contains barriers: every thread of the
// workgroup must call it.
template <int BLOCK, typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* lds, T* total) {
    constexpr int NW = BLOCK / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    T inc = wave_inclusive_scan(v);
    if (lane == kWave - 1) lds[wid] = inc;
    __syncthreads();
    T wave_off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        T x = lds[w];
        if (w < wid) wave_off += x;
        tot += x;
    }
    __syncthreads();
    *total = tot;
    return wave_off + inc - v;
}

// Non-temporal (streaming) loads for data read exactly once.
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {
    return __builtin_nontemporal_load(p);
}

}  // namespace tg
