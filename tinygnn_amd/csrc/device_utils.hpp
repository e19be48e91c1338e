// device_utils.hpp -- wave64 / workgroup primitives for gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

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

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Lane SRC of the caller's group of LPR consecutive lanes (groups aligned to
// LPR), to every lane of the group.  16- and 4-lane groups use one DPP
// move (row broadcast within a 16-lane row, quad permute), with no LDS
// traffic: the config-E GAT passes (16-lane groups) ran 1.5% faster than
// with ds_bpermute.  Other widths keep the shuffle: two DPP moves and a
// select for 8 lanes were no faster, and readlane for 32 lanes made the
// F=128 SpMM 0.8% slower.  Every lane of the caller's group must be
// active; lanes of other groups may not be.
template <int LPR, int SRC>
__device__ __forceinline__ int group_bcast(int v) {
    static_assert(SRC >= 0 && SRC < LPR, "source lane outside the group");
    // every lane of the row or quad is written: no old value (mov_dpp)
    if constexpr (LPR == 16) {
        return __builtin_amdgcn_mov_dpp(v, 0x150 + SRC, 0xF, 0xF, false);  // row_newbcast
    } else if constexpr (LPR == 4) {
        return __builtin_amdgcn_mov_dpp(v, SRC | (SRC << 2) | (SRC << 4) | (SRC << 6), 0xF, 0xF,
                                        false);  // quad_perm
    } else {
        return __shfl(v, SRC, LPR);
    }
}

template <int LPR, int SRC>
__device__ __forceinline__ float group_bcast(float v) {
    return __int_as_float(group_bcast<LPR, SRC>(__float_as_int(v)));
}

// The value of the partner lane that differs in lane bit K (K = 8, 4, 2, 1)
// within a 16-lane row, and in no higher bit: row_mirror (lane i <-> 15 - i)
// for 8, row_half_mirror (i <-> 7 - i within each eight) for 4, quad_perm
// [2,3,0,1] and [1,0,3,2] for 2 and 1.  The partner must be active.  (With
// an old value the compiler folds the move into a following add, v_add_dpp.)
template <int K>
__device__ __forceinline__ float dpp_flip(float v) {
    static_assert(K == 8 || K == 4 || K == 2 || K == 1, "partner bit");
    constexpr int ctrl = K == 8 ? 0x140 : K == 4 ? 0x141 : K == 2 ? 0x4E : 0xB1;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

template <int K, int N>
__device__ __forceinline__ void transpose_sum_step(float* x, int lane) {
    // x[0, N) -> x[0, N / 2): the half that lane bit K selects, plus the
    // partner's copy of it (the partner keeps the other half)
    const bool hi = (lane & K) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float a = x[i], b = x[i + N / 2];
        const float send = hi ? a : b;
        const float keep = hi ? b : a;
        x[i] = keep + dpp_flip<K>(send);
    }
    if constexpr (K > 1) transpose_sum_step<K / 2, N / 2>(x, lane);
}

// Sums x[u] over the LPR lanes of a group (LPR 8 or 16, groups aligned to
// LPR lanes, all active): on return x[j], j < N / LPR, of lane l holds the
// total of entry l * (N / LPR) + j.  log2(LPR) halving steps, N - N / LPR
// adds per lane, no LDS; each total is one fixed tree of adds.
template <int LPR, int N>
__device__ __forceinline__ void group_transpose_sum(float (&x)[N], int lane) {
    static_assert((LPR == 8 || LPR == 16) && N % LPR == 0, "group shape");
    transpose_sum_step<LPR / 2, N>(x, lane);
}

// v with lane LANE replaced by the wave-uniform value s (v_writelane_b32;
// this compiler has no builtin for it).
template <int LANE>
__device__ __forceinline__ uint32_t write_lane(uint32_t s, uint32_t v) {
    static_assert(LANE >= 0 && LANE < kWave, "lane");
    asm("v_writelane_b32 %0, %1, %2" : "=v"(v) : "s"(s), "i"(LANE), "0"(v));
    return v;
}

// Non-temporal (streaming) loads for data read exactly once.
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {
    return __builtin_nontemporal_load(p);
}

}  // namespace tg
