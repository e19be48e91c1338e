// dense.hip -- dense transforms and epilogues for gfx950.
//
// Replaces tinygnn::matmul (reference src/ops.cpp:70-162) and the in-place
// epilogues (ops.cpp:328-661): relu, leaky_relu, elu, sigmoid, tanh, gelu,
// softmax, log_softmax, add_bias, plus edge_softmax (src/layers.cpp:768-822).
//
// Two GEMMs:
//   * in order: one fma chain per output over k ascending from 0, through
//     LDS tiles -- bit-identical to the reference; used for thin outputs
//     (F_out 7/16/41) where the product is not a real contraction;
//   * MFMA: v_mfma_f32_16x16x4f32, 128x128 workgroup tiles of four 64x64
//     wavefront tiles, for the wide transforms (602->256, 4 heads x 64).
// Both fuse the bias add and the activation into the store.
#include "common.hpp"
#include "dense.hpp"
#include "device_utils.hpp"

#include <string>

namespace tg {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
// 128-bit loads at any dword address (gfx950's global loads take them
// unaligned)
typedef float Float4Dw __attribute__((ext_vector_type(4), aligned(4)));

// Element (m, n) of the output, row-major or tile-major (GemmArgs).
__device__ __forceinline__ int64_t c_index(const GemmArgs& g, int64_t m, int64_t n) {
    return g.c_tile_stride > 0 ? (n >> 5) * g.c_tile_stride + m * 32 + (n & 31) : m * g.ldc + n;
}

__device__ __forceinline__ float epi_apply(float x, const float* __restrict__ bias, int64_t n,
                                           int epi) {
    if (bias) x = x + bias[n];
    if (epi == TG_EPI_RELU) {
        x = (0.0f < x) ? x : 0.0f;
    } else if (epi == TG_EPI_ELU) {
        if (x < 0.0f) x = 1.0f * (expf(x) - 1.0f);
    }
    return x;
}

// Output element (m, n): the row factor, then bias and activation.
__device__ __forceinline__ float epi_out(const GemmArgs& g, float x, int64_t m, int64_t n) {
    if (g.row_scale) x = x * g.row_scale[m];
    return epi_apply(x, g.bias, n, g.epi);
}

// epi_apply's activation with the epilogue fixed at compile time.
template <int EPI>
__device__ __forceinline__ float epi_act(float x) {
    if (EPI == TG_EPI_RELU) return (0.0f < x) ? x : 0.0f;
    if (EPI == TG_EPI_ELU) return (x < 0.0f) ? 1.0f * (expf(x) - 1.0f) : x;
    return x;
}

// Stores one lane's outputs of MI x NJ 16x16 MFMA tiles (D layout of
// v_mfma_f32_16x16x4f32: lane (q, r) holds rows 4q..4q+3 of column r), the
// tiles' rows from mb, columns from nb: C[m][n] = EPI(acc * row_scale[m] +
// bias[n]) as epi_out computes it, C tile-major (TILED) or row-major.  The
// row factors and bias terms are loaded before the first store: C may alias
// them as far as the compiler knows, so loads between the stores would each
// wait for a round trip.  A missing row factor is 1 (x * 1 = x exactly), and
// the store loop has no branch but the bounds.  (Per-element loads and
// epilogue branches cost 6% of the config-E layer-1 transform, one index
// formula for both layouts with a run-time row stride another 2.5%.)
template <int EPI, bool TILED, int MI, int NJ>
__device__ __forceinline__ void store_tiles(const GemmArgs& g, const v4f (&acc)[MI][NJ],
                                            int64_t mb, int64_t nb, int q, int r) {
    float rsv[MI][4], bv[NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int64_t m = mb + i * 16 + 4 * q + rr;
            rsv[i][rr] = (g.row_scale && m < g.m) ? g.row_scale[m] : 1.0f;
        }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int64_t n = nb + j * 16 + r;
        bv[j] = (g.bias && n < g.n) ? g.bias[n] : 0.0f;
    }
    const bool has_bias = g.bias != nullptr;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int64_t gn = nb + j * 16 + r;
            if (gn >= g.n) continue;
            float* cc = TILED ? g.c + (gn >> 5) * g.c_tile_stride + (gn & 31) : g.c + gn;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int64_t m = mb + i * 16 + 4 * q + rr;
                if (m >= g.m) continue;
                float x = acc[i][j][rr] * rsv[i][rr];
                if (has_bias) x = x + bv[j];
                cc[TILED ? m * 32 : m * g.ldc] = epi_act<EPI>(x);
            }
        }
}

// store_tiles for C's layout (GemmArgs::c_tile_stride).
template <int EPI, int MI, int NJ>
__device__ __forceinline__ void store_tiles_c(const GemmArgs& g, const v4f (&acc)[MI][NJ],
                                              int64_t mb, int64_t nb, int q, int r) {
    if (g.c_tile_stride > 0)
        store_tiles<EPI, true>(g, acc, mb, nb, q, r);
    else
        store_tiles<EPI, false>(g, acc, mb, nb, q, r);
}

// store_tiles with the epilogue chosen at run time (one of three bodies runs).
template <int MI, int NJ>
__device__ __forceinline__ void store_tiles_any(const GemmArgs& g, const v4f (&acc)[MI][NJ],
                                                int64_t mb, int64_t nb, int q, int r) {
    if (g.epi == TG_EPI_RELU)
        store_tiles_c<TG_EPI_RELU>(g, acc, mb, nb, q, r);
    else if (g.epi == TG_EPI_ELU)
        store_tiles_c<TG_EPI_ELU>(g, acc, mb, nb, q, r);
    else
        store_tiles_c<TG_EPI_NONE>(g, acc, mb, nb, q, r);
}

// ---------------------------------------------------------------------------
// In-order GEMM (bit-exact)
// ---------------------------------------------------------------------------
template <int BM, int BN, int TM, int TN, bool DUAL>
__global__ __launch_bounds__(256) void gemm_inorder_kernel(GemmArgs g) {
    constexpr int BK = 16;
    constexpr int TX = BN / TN;
    constexpr int TY = BM / TM;
    static_assert(TX * TY == 256, "256 threads");
    constexpr int NP = DUAL ? 2 : 1;
    __shared__ float As[NP][BK][BM];
    __shared__ float Bs[NP][BK][BN];
    const int tx = threadIdx.x % TX;
    const int ty = threadIdx.x / TX;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * BM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.y) * BN;
    const int64_t M = g.m, N = g.n, K = g.k1;

    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;

    // tail columns (dual only): tail_from is a multiple of 8, so a thread's
    // TN consecutive columns are all tail or all not
    const bool tail = DUAL && g.tail_from >= 0 && (n0 + tx * TN) >= g.tail_from;

    for (int64_t k0 = 0; k0 < K; k0 += BK) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float* A = p ? g.a2 : g.a1;
            const float* B = p ? g.b2 : g.b1;
            const int64_t lda = p ? g.lda2 : g.lda1;
            const int64_t ldb = p ? g.ldb2 : g.ldb1;
            for (int e = threadIdx.x; e < BM * BK; e += 256) {
                const int mm = e / BK, kk = e % BK;
                const int64_t gm = m0 + mm, gk = k0 + kk;
                As[p][kk][mm] = (gm < M && gk < K) ? A[gm * lda + gk] : 0.0f;
            }
            for (int e = threadIdx.x; e < BN * BK; e += 256) {
                const int kk = e / BN, nn = e % BN;
                const int64_t gk = k0 + kk, gn = n0 + nn;
                Bs[p][kk][nn] = (gk < K && gn < N) ? B[gk * ldb + gn] : 0.0f;
            }
        }
        __syncthreads();
        const int kmax = static_cast<int>(K - k0 < BK ? K - k0 : BK);
        for (int kk = 0; kk < kmax; ++kk) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = As[0][kk][ty * TM + i];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = Bs[0][kk][tx * TN + j];
            if constexpr (DUAL) {
                float a2[TM], b2[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) a2[i] = As[NP - 1][kk][ty * TM + i];
#pragma unroll
                for (int j = 0; j < TN; ++j) b2[j] = Bs[NP - 1][kk][tx * TN + j];
                if (tail) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            acc[i][j] = acc[i][j] + __builtin_fmaf(a[i], b[j], a2[i] * b2[j]);
                } else {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const float t = __builtin_fmaf(a[i], b[j], acc[i][j]);
                            acc[i][j] = __builtin_fmaf(a2[i], b2[j], t);
                        }
                }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int64_t gm = m0 + ty * TM + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t gn = n0 + tx * TN + j;
            if (gn < N) g.c[c_index(g, gm, gn)] = epi_out(g, acc[i][j], gm, gn);
        }
    }
}

// ---------------------------------------------------------------------------
// In-order GEMM for small products (bit-exact; m n <= 2^21, e.g. the
// Cora-scale transforms): one output per thread, a workgroup covers BM x BN
// outputs (BM = 256 / BN), so a 2,708-row product gets 170-680 workgroups
// instead of 11-22, and the k loop runs over 64-wide tiles with the next
// tile loaded into registers while the current one is consumed from LDS.
// Each output is one fma chain over k ascending from 0 (padded k is never
// accumulated); DUAL interleaves the pairs per k and applies the scalar tail
// exactly as gemm_inorder_kernel.
// ---------------------------------------------------------------------------
constexpr int kSBK = 64;

template <int BN, bool DUAL>
__global__ __launch_bounds__(256) void gemm_inorder_small_kernel(GemmArgs g) {
    constexpr int BM = 256 / BN;
    constexpr int NP = DUAL ? 2 : 1;
    constexpr int LA = BM * kSBK / 256;  // A values per thread per tile
    constexpr int LB = kSBK * BN / 256;  // B values per thread per tile
    static_assert(LA >= 1 && LB >= 1, "tile shape");
    __shared__ float As[2][NP][kSBK][BM];
    __shared__ float Bs[2][NP][kSBK][BN];
    const int tx = threadIdx.x % BN, ty = threadIdx.x / BN;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * BM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.y) * BN;
    const int64_t M = g.m, N = g.n, K = g.k1;
    const int64_t nt = (K + kSBK - 1) / kSBK;
    const bool tail = DUAL && g.tail_from >= 0 && (n0 + tx) >= g.tail_from;

    float ra[NP][LA], rb[NP][LB];
    auto fetch = [&](int64_t kt) {
        const int64_t k0 = kt * kSBK;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float* A = p ? g.a2 : g.a1;
            const float* B = p ? g.b2 : g.b1;
            const int64_t lda = p ? g.lda2 : g.lda1;
            const int64_t ldb = p ? g.ldb2 : g.ldb1;
#pragma unroll
            for (int t = 0; t < LA; ++t) {
                const int e = threadIdx.x + 256 * t;
                const int64_t gm = m0 + e / kSBK, gk = k0 + e % kSBK;
                ra[p][t] = (gm < M && gk < K) ? A[gm * lda + gk] : 0.0f;
            }
#pragma unroll
            for (int t = 0; t < LB; ++t) {
                const int e = threadIdx.x + 256 * t;
                const int64_t gk = k0 + e / BN, gn = n0 + e % BN;
                rb[p][t] = (gk < K && gn < N) ? B[gk * ldb + gn] : 0.0f;
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int t = 0; t < LA; ++t) {
                const int e = threadIdx.x + 256 * t;
                As[buf][p][e % kSBK][e / kSBK] = ra[p][t];
            }
#pragma unroll
            for (int t = 0; t < LB; ++t) {
                const int e = threadIdx.x + 256 * t;
                Bs[buf][p][e / BN][e % BN] = rb[p][t];
            }
        }
    };

    float acc = 0.0f;
    if (nt > 0) {
        fetch(0);
        stage(0);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nt; ++kt) {
        const int cb = static_cast<int>(kt & 1);
        if (kt + 1 < nt) fetch(kt + 1);
        const int64_t k0 = kt * kSBK;
        const int kmax = static_cast<int>(K - k0 < kSBK ? K - k0 : kSBK);
        // the dual form is chosen outside the k loop (a branch inside it
        // cost Cora-scale dual n x 1433 x 64 about a third of its time)
        if (DUAL && tail) {
            for (int kk = 0; kk < kmax; ++kk) {
                const float a = As[cb][0][kk][ty], b = Bs[cb][0][kk][tx];
                const float a2 = As[cb][NP - 1][kk][ty], b2 = Bs[cb][NP - 1][kk][tx];
                acc = acc + __builtin_fmaf(a, b, a2 * b2);
            }
        } else {
            for (int kk = 0; kk < kmax; ++kk) {
                const float a = As[cb][0][kk][ty], b = Bs[cb][0][kk][tx];
                if constexpr (DUAL) {
                    const float a2 = As[cb][NP - 1][kk][ty], b2 = Bs[cb][NP - 1][kk][tx];
                    acc = __builtin_fmaf(a2, b2, __builtin_fmaf(a, b, acc));
                } else {
                    acc = __builtin_fmaf(a, b, acc);
                }
            }
        }
        if (kt + 1 < nt) stage(cb ^ 1);
        __syncthreads();
    }
    const int64_t gm = m0 + ty, gn = n0 + tx;
    if (gm < M && gn < N) g.c[c_index(g, gm, gn)] = epi_out(g, acc, gm, gn);
}

// ---------------------------------------------------------------------------
// In-order GEMM for small products in 64-column slabs (bit-exact; the
// Cora-scale dual n x 1433 x 64 SAGE transform): a wavefront computes TM
// rows x 64 columns, one column per lane.  The rows are wave-uniform, so
// their A values come through scalar loads (s_load_dwordx16, no LDS); the
// workgroup's four wavefronts share each k-tile of kRKT rows of B through
// LDS (two buffers, the next tile loaded into registers while the current
// one is consumed).  Every output is one fma chain over k ascending from
// 0, never over padded k; DUAL interleaves the pairs per k and applies the
// reference's scalar tail, as gemm_inorder_kernel.  A tile's A values (TM x
// kRKT per pair) must fit the scalar registers.  Measured on the dual
// 2708 x 1433 x 64 product (Cora-synth SAGE forward, 204 us with
// gemm_inorder_small_kernel): TM 1 / kRKT 32 145 us, kRKT 16 154 us, kRKT
// 64 200 us (scalar spills), TM 2 169 us, TM 4 255 us; the single product
// (GAT) is no faster than gemm_inorder_small_kernel and stays there.
// ---------------------------------------------------------------------------
template <int TM, int kRKT, bool DUAL>
__global__ __launch_bounds__(256) void gemm_inorder_rows_kernel(GemmArgs g) {
    constexpr int NP = DUAL ? 2 : 1;
    constexpr int LB = kRKT * 64 / 256;  // B values per thread per tile and pair
    __shared__ float Bs[2][NP][kRKT][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t M = g.m, N = g.n, K = g.k1;
    const int64_t n0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * TM;
    const int64_t nt = (K + kRKT - 1) / kRKT;
    // the wave's rows of A (clamped for the loads; rows >= M are not stored)
    const float* ar[NP][TM];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int r = 0; r < TM; ++r) {
            const int64_t row = m0 + r < M ? m0 + r : M - 1;
            ar[p][r] = p ? g.a2 + row * g.lda2 : g.a1 + row * g.lda1;
        }
    const bool tail = DUAL && g.tail_from >= 0 && (n0 + lane) >= g.tail_from;

    float rb[NP][LB];
    auto fetch = [&](int64_t kt) {
        const int64_t k0 = kt * kRKT;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float* B = p ? g.b2 : g.b1;
            const int64_t ldb = p ? g.ldb2 : g.ldb1;
#pragma unroll
            for (int t = 0; t < LB; ++t) {
                const int e = threadIdx.x + 256 * t;
                const int64_t gk = k0 + e / 64, gn = n0 + e % 64;
                rb[p][t] = (gk < K && gn < N) ? B[gk * ldb + gn] : 0.0f;
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int t = 0; t < LB; ++t) {
                const int e = threadIdx.x + 256 * t;
                Bs[buf][p][e / 64][e % 64] = rb[p][t];
            }
    };

    float acc[TM];
#pragma unroll
    for (int r = 0; r < TM; ++r) acc[r] = 0.0f;
    // one k step of every row: plain (tail = false) or the scalar tail form
    auto step = [&](int cb, int64_t k, int kk, bool tl) {
        const float b1 = Bs[cb][0][kk][lane];
        const float b2 = Bs[cb][NP - 1][kk][lane];
#pragma unroll
        for (int r = 0; r < TM; ++r) {
            const float a1 = ar[0][r][k];
            if constexpr (DUAL) {
                const float a2 = ar[NP - 1][r][k];
                acc[r] = tl ? acc[r] + __builtin_fmaf(a1, b1, a2 * b2)
                            : __builtin_fmaf(a2, b2, __builtin_fmaf(a1, b1, acc[r]));
            } else {
                acc[r] = __builtin_fmaf(a1, b1, acc[r]);
            }
        }
    };
    if (nt > 0) {
        fetch(0);
        stage(0);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nt; ++kt) {
        const int cb = static_cast<int>(kt & 1);
        if (kt + 1 < nt) fetch(kt + 1);
        const int64_t k0 = kt * kRKT;
        const int kmax = static_cast<int>(K - k0 < kRKT ? K - k0 : kRKT);
        // the dual form is chosen outside the k loop
        if (kmax == kRKT) {
            if (DUAL && tail) {
#pragma unroll
                for (int kk = 0; kk < kRKT; ++kk) step(cb, k0 + kk, kk, true);
            } else {
#pragma unroll
                for (int kk = 0; kk < kRKT; ++kk) step(cb, k0 + kk, kk, false);
            }
        } else {
            if (DUAL && tail) {
                for (int kk = 0; kk < kmax; ++kk) step(cb, k0 + kk, kk, true);
            } else {
                for (int kk = 0; kk < kmax; ++kk) step(cb, k0 + kk, kk, false);
            }
        }
        if (kt + 1 < nt) stage(cb ^ 1);
        __syncthreads();
    }
    const int64_t gn = n0 + lane;
#pragma unroll
    for (int r = 0; r < TM; ++r) {
        const int64_t gm = m0 + r;
        if (gm < M && gn < N) g.c[c_index(g, gm, gn)] = epi_out(g, acc[r], gm, gn);
    }
}

// ---------------------------------------------------------------------------
// Wide in-order GEMM (bit-exact, n > 32): 128x128 workgroup tile, an 8x8
// register micro-tile per thread, BK = 8, two LDS buffers with register
// prefetch.  Each output is still one fma chain over k ascending from 0 (the
// k loop is outermost, and no padded k is ever accumulated), so the result
// equals the reference's (i,k,j) loop bit for bit; DUAL interleaves the two
// products per k exactly as the in-order kernel above.
// ---------------------------------------------------------------------------
constexpr int kWBM = 128, kWBN = 128, kWBK = 8;

template <int VA, bool DUAL>
__global__ __launch_bounds__(256) void gemm_inorder_wide_kernel(GemmArgs g) {
    constexpr int NP = DUAL ? 2 : 1;
    __shared__ __attribute__((aligned(16))) float As[2][NP][kWBK][kWBM];
    __shared__ __attribute__((aligned(16))) float Bs[2][NP][kWBK][kWBN];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kWBM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.y) * kWBN;
    const int64_t M = g.m, N = g.n, K = g.k1;
    const int64_t nt = (K + kWBK - 1) / kWBK;
    // loads: A row ar, 4 k from ak; B row bk, 4 n from bn
    const int ar = threadIdx.x >> 1, ak = (threadIdx.x & 1) * 4;
    const int bk = threadIdx.x >> 5, bn = (threadIdx.x & 31) * 4;
    float ra[NP][4], rb[NP][4];

    auto fetch = [&](int64_t kt) {
        const int64_t k0 = kt * kWBK;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float* A = p ? g.a2 : g.a1;
            const float* B = p ? g.b2 : g.b1;
            const int64_t lda = p ? g.lda2 : g.lda1;
            const int64_t ldb = p ? g.ldb2 : g.ldb1;
            const int64_t gm = m0 + ar, ka = k0 + ak;
            const float* pa = A + (gm < M ? gm : 0) * lda + ka;
            const int64_t va = gm < M ? K - ka : 0;
            if (VA == 4 && va >= 4) {
                const Float4Dw t = *reinterpret_cast<const Float4Dw*>(pa);
                ra[p][0] = t.x; ra[p][1] = t.y; ra[p][2] = t.z; ra[p][3] = t.w;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) ra[p][u] = u < va ? pa[u] : 0.0f;
            }
            const int64_t kb = k0 + bk, nb = n0 + bn;
            const float* pb = B + (kb < K ? kb : 0) * ldb + nb;
            const int64_t vb = kb < K ? N - nb : 0;
            if (vb >= 4) {
                const Float4Dw t = *reinterpret_cast<const Float4Dw*>(pb);
                rb[p][0] = t.x; rb[p][1] = t.y; rb[p][2] = t.z; rb[p][3] = t.w;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) rb[p][u] = u < vb ? pb[u] : 0.0f;
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int u = 0; u < 4; ++u) As[buf][p][ak + u][ar] = ra[p][u];
            *reinterpret_cast<float4*>(&Bs[buf][p][bk][bn]) =
                make_float4(rb[p][0], rb[p][1], rb[p][2], rb[p][3]);
        }
    };

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
    // tail columns (dual only): tail_from is a multiple of 8, so a thread's
    // eight consecutive columns are all tail or all not
    const bool tail = DUAL && g.tail_from >= 0 && (n0 + tx * 8) >= g.tail_from;

    if (nt > 0) {
        fetch(0);
        stage(0);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nt; ++kt) {
        const int cb = static_cast<int>(kt & 1);
        if (kt + 1 < nt) fetch(kt + 1);
        const int kmax = static_cast<int>(K - kt * kWBK < kWBK ? K - kt * kWBK : kWBK);
        for (int kk = 0; kk < kmax; ++kk) {
            float a[NP][8], b[NP][8];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float4 a0 = *reinterpret_cast<const float4*>(&As[cb][p][kk][ty * 8]);
                const float4 a1 = *reinterpret_cast<const float4*>(&As[cb][p][kk][ty * 8 + 4]);
                const float4 b0 = *reinterpret_cast<const float4*>(&Bs[cb][p][kk][tx * 8]);
                const float4 b1 = *reinterpret_cast<const float4*>(&Bs[cb][p][kk][tx * 8 + 4]);
                a[p][0] = a0.x; a[p][1] = a0.y; a[p][2] = a0.z; a[p][3] = a0.w;
                a[p][4] = a1.x; a[p][5] = a1.y; a[p][6] = a1.z; a[p][7] = a1.w;
                b[p][0] = b0.x; b[p][1] = b0.y; b[p][2] = b0.z; b[p][3] = b0.w;
                b[p][4] = b1.x; b[p][5] = b1.y; b[p][6] = b1.z; b[p][7] = b1.w;
            }
            if constexpr (DUAL) {
                if (tail) {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            acc[i][j] = acc[i][j] +
                                        __builtin_fmaf(a[0][i], b[0][j], a[NP - 1][i] * b[NP - 1][j]);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const float t = __builtin_fmaf(a[0][i], b[0][j], acc[i][j]);
                            acc[i][j] = __builtin_fmaf(a[NP - 1][i], b[NP - 1][j], t);
                        }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        acc[i][j] = __builtin_fmaf(a[0][i], b[0][j], acc[i][j]);
            }
        }
        if (kt + 1 < nt) stage(cb ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t gm = m0 + ty * 8 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t gn = n0 + tx * 8 + j;
            if (gn < N) g.c[c_index(g, gm, gn)] = epi_out(g, acc[i][j], gm, gn);
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM: 128x128 workgroup tile, 2x2 wavefronts of 64x64 (4x4 tiles of
// v_mfma_f32_16x16x4f32), BK = 16, two LDS buffers with register prefetch:
// the next K tile is loaded from global memory while the current one feeds
// the MFMAs, so there is one barrier per tile.
// Lane (q = lane/16, r = lane%16) feeds k = 4q + s at MFMA step s for both
// operands (the products pair up; only the order of the k sum changes).
// A is staged as [m][k] so a lane's four k values of a row are one 128-bit
// LDS read; B stays [k][n] and is read 32 bits at a time.
// LDS layouts, measured free of bank conflicts on gfx950 (SQ_LDS_BANK_CONFLICT
// = 0): A rows at a 24-float pitch, read by 16 rows x 4 chunks per
// wavefront step, written by each 16 lanes as 8 rows x 2 chunks (the 16
// chunk addresses cover the 64 banks once); B rows at a 132-float pitch,
// written 16 lanes per row as 256 contiguous bytes.  (A at a 20-float pitch,
// 2 lanes per row, and B at 8 columns per lane each cost a 2-way conflict:
// 29% of LDS cycles.)
// ---------------------------------------------------------------------------
constexpr int kMBM = 128, kMBN = 128, kMBK = 16;
constexpr int kMLDA = kMBK + 8;   // A tile pitch (floats)
constexpr int kMLDB = kMBN + 4;   // B tile pitch

// Loads p[0..3] of which the first `valid` exist (valid <= 0: none) as one
// 128-bit access when all 4 exist and V = 4.  gfx950's global loads take a
// 128-bit access at any dword address (config-E transform, 602-float rows of
// A at 8-byte alignment: 128-bit loads 0.68 ms, 64-bit 0.72 ms).
template <int V>
__device__ __forceinline__ v4f load4(const float* __restrict__ p, int64_t valid) {
    if (V == 4 && valid >= 4) return *reinterpret_cast<const Float4Dw*>(p);
    v4f x;
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = (u < valid) ? p[u] : 0.0f;
    return x;
}

// VA / VB: 4 = 128-bit operand loads (dword-aligned pointers), 1 = 32-bit.
// EPI: g.epi.  Launch bound (256, 3): three workgroups per CU (41.5 KB of
// LDS each) need at most 168 registers per lane.
template <int VA, int VB, int EPI>
__global__ __launch_bounds__(256, 3) void gemm_mfma_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) float As[2][kMBM][kMLDA];
    __shared__ __attribute__((aligned(16))) float Bs[2][kMBK][kMLDB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int q = lane >> 4, r = lane & 15;
    const int64_t M = g.m, N = g.n;
    // Workgroup i runs on XCD i % 8 (round-robin dispatch).  XCD x takes the
    // row tiles m = x (mod 8), and for each of them its column tiles one
    // after another, so the second and later reads of the row tile's A
    // find it in that XCD's L2.  Ids past an XCD's tiles exit.
    const int64_t mt = (M + kMBM - 1) / kMBM, ntl = (N + kMBN - 1) / kMBN;
    const int64_t xj = blockIdx.x / 8;
    const int64_t mtile = (xj / ntl) * 8 + blockIdx.x % 8;
    if (mtile >= mt) return;  // before any barrier: the whole workgroup
    const int64_t m0 = mtile * kMBM;
    const int64_t n0 = (xj % ntl) * kMBN;
    const int64_t t1 = (g.k1 + kMBK - 1) / kMBK;
    const int64_t nt = t1 + (g.a2 ? (g.k2 + kMBK - 1) / kMBK : 0);

    // This thread's share of a tile: A row ar, k chunks ac and ac + 2 (4
    // floats each); B row bkr, column chunks bc and bc + 16.  Rows past M
    // read row M - 1 (their outputs are not stored), so a tile whose k range
    // is whole loads A without guards.
    const int ar = threadIdx.x >> 1, ac = threadIdx.x & 1;
    const int bkr = threadIdx.x >> 4, bc = threadIdx.x & 15;
    const int64_t gm = m0 + ar;
    const int64_t gmc = gm < M ? gm : M - 1;
    const int64_t nb0 = n0 + 4 * bc, nb1 = nb0 + 64;
    const bool colfull = n0 + kMBN <= N;  // uniform
    const float* pa1 = g.a1 ? g.a1 + gmc * g.lda1 + 4 * ac : nullptr;
    const float* pa2 = g.a2 ? g.a2 + gmc * g.lda2 + 4 * ac : nullptr;
    const float* pb1 = g.b1 ? g.b1 + bkr * g.ldb1 : nullptr;
    const float* pb2 = g.b2 ? g.b2 + bkr * g.ldb2 : nullptr;
    v4f ra0, ra1, rb0, rb1;

    auto fetch = [&](int64_t kt) {
        const bool seg2 = kt >= t1;  // uniform, as is everything but the lanes' rows
        const int64_t ldb = seg2 ? g.ldb2 : g.ldb1;
        const int64_t K = seg2 ? g.k2 : g.k1;
        const int64_t k0 = (seg2 ? kt - t1 : kt) * kMBK;
        const float* pa = (seg2 ? pa2 : pa1) + k0;
        if (k0 + kMBK <= K) {  // whole k range
            const float* pb = (seg2 ? pb2 : pb1) + k0 * ldb;
            ra0 = load4<VA>(pa, 4);
            ra1 = load4<VA>(pa + 8, 4);
            if (colfull) {
                rb0 = load4<VB>(pb + nb0, 4);
                rb1 = load4<VB>(pb + nb1, 4);
            } else {
                rb0 = load4<VB>(pb + nb0, N - nb0);
                rb1 = load4<VB>(pb + nb1, N - nb1);
            }
        } else {
            const int64_t kb = k0 + bkr;
            const float* pb = kb < K ? (seg2 ? pb2 : pb1) + k0 * ldb : (seg2 ? g.b2 : g.b1);
            const int64_t ka = k0 + 4 * ac;
            ra0 = load4<1>(pa, gm < M ? K - ka : 0);
            ra1 = load4<1>(pa + 8, gm < M ? K - ka - 8 : 0);
            rb0 = load4<1>(pb + nb0, kb < K ? N - nb0 : 0);
            rb1 = load4<1>(pb + nb1, kb < K ? N - nb1 : 0);
        }
    };
    auto stage = [&](int buf) {
        *reinterpret_cast<v4f*>(&As[buf][ar][4 * ac]) = ra0;
        *reinterpret_cast<v4f*>(&As[buf][ar][4 * ac + 8]) = ra1;
        *reinterpret_cast<v4f*>(&Bs[buf][bkr][4 * bc]) = rb0;
        *reinterpret_cast<v4f*>(&Bs[buf][bkr][4 * bc + 64]) = rb1;
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    if (nt > 0) {
        fetch(0);
        stage(0);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nt; ++kt) {
        const int cb = static_cast<int>(kt & 1);
        if (kt + 1 < nt) fetch(kt + 1);
        // keep the next tile's loads ahead of this tile's MFMAs (left to
        // itself the scheduler sinks them below, exposing their latency)
        __builtin_amdgcn_sched_barrier(0);
        v4f a[4];
        float b[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4f*>(&As[cb][wm + i * 16 + r][4 * q]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) b[j][s] = Bs[cb][4 * q + s][wn + j * 16 + r];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s], b[j][s], acc[i][j],
                                                                     0, 0, 0);
        if (kt + 1 < nt) stage(cb ^ 1);
        __syncthreads();
    }
    store_tiles_c<EPI>(g, acc, m0 + wm, n0 + wn, q, r);
}

// ---------------------------------------------------------------------------
// Thin MFMA GEMM (n <= 64): each wavefront owns 64 rows x 16 NT columns
// (4 x NT tiles of v_mfma_f32_16x16x4f32) and reads its operands straight
// from global memory in the MFMA layout, with no LDS and no barrier.  In a
// chunk of 32 k values lane (q, r) feeds k = k0 + 8q + s at MFMA step s
// (s = 0..7) for both operands, so its A values of a row are 8 consecutive
// floats (two 128-bit loads; the wavefront reads whole 128-byte lines) and
// its B values are column 16 j + r of rows k0 + 8q .. k0 + 8q + 7 (B is a
// few KB and stays in L1/L2).  The next chunk's operands are loaded while
// the current chunk's MFMAs run.  A 128 x 128 tile would do 128/n times the
// needed MFMA work at n = 41; here it is 16 NT / n (48 / 41).
// ---------------------------------------------------------------------------
constexpr int kTK = 32;  // k per chunk

template <int NT, bool ALIGNED>
__global__ __launch_bounds__(256) void gemm_mfma_thin_kernel(GemmArgs g) {
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4, r = lane & 15;
    const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 64;
    const int64_t M = g.m, N = g.n;
    if (m0 >= M) return;  // no barrier in this kernel: waves retire independently
    const int64_t t1 = (g.k1 + kTK - 1) / kTK;
    const int64_t nt = t1 + (g.a2 ? (g.k2 + kTK - 1) / kTK : 0);

    float a[4][8], b[NT][8];
    auto fetch = [&](int64_t kt, float (&ra)[4][8], float (&rb)[NT][8]) {
        const bool seg2 = kt >= t1;
        const float* A = seg2 ? g.a2 : g.a1;
        const float* B = seg2 ? g.b2 : g.b1;
        const int64_t lda = seg2 ? g.lda2 : g.lda1;
        const int64_t ldb = seg2 ? g.ldb2 : g.ldb1;
        const int64_t K = seg2 ? g.k2 : g.k1;
        const int64_t k = (seg2 ? kt - t1 : kt) * kTK + 8 * q;  // this lane's first k
        const int64_t kv = K - k;  // valid k values from k on (may be <= 0)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t gm = m0 + 16 * i + r;
            const float* p = A + (gm < M ? gm : 0) * lda + (kv > 0 ? k : 0);
            if (ALIGNED && gm < M && kv >= 8) {
                const Float4Dw x0 = *reinterpret_cast<const Float4Dw*>(p);
                const Float4Dw x1 = *reinterpret_cast<const Float4Dw*>(p + 4);
                ra[i][0] = x0.x; ra[i][1] = x0.y; ra[i][2] = x0.z; ra[i][3] = x0.w;
                ra[i][4] = x1.x; ra[i][5] = x1.y; ra[i][6] = x1.z; ra[i][7] = x1.w;
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) ra[i][t] = (gm < M && t < kv) ? p[t] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int64_t gn = 16 * j + r;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                rb[j][t] = (gn < N && t < kv) ? B[(k + t) * ldb + gn] : 0.0f;
        }
    };

    v4f acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (nt > 0) fetch(0, a, b);
    for (int64_t kt = 0; kt < nt; ++kt) {
        float na[4][8], nb[NT][8];
        if (kt + 1 < nt) fetch(kt + 1, na, nb);
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s], b[j][s], acc[i][j],
                                                                     0, 0, 0);
        if (kt + 1 < nt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int t = 0; t < 8; ++t) a[i][t] = na[i][t];
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int t = 0; t < 8; ++t) b[j][t] = nb[j][t];
        }
    }
    store_tiles_any(g, acc, m0, 0, q, r);
}

// Thin MFMA GEMM with B in LDS (one pair, n <= 64, round_up(k, 32) x 16 NT
// floats of B <= 64 KB): B is staged once per workgroup, packed so that a
// lane's 8 k values of its column are two 128-bit LDS reads; each wavefront
// owns 32 rows (2 x NT tiles) and keeps A two chunks ahead in registers, so
// more waves and more bytes are in flight than with B in registers.
constexpr int kThinRows = 32;                  // rows per wavefront
constexpr int kThinWaves = 8;                  // wavefronts per workgroup
constexpr int64_t kThinLdsFloats = 16 * 1024;  // B panel budget (64 KB)

template <int NT>
__global__ __launch_bounds__(512) void gemm_mfma_thin_lds_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) float Bs[];  // [k/8][16 NT][8]
    constexpr int BN = 16 * NT;
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4, r = lane & 15;
    const int64_t M = g.m, N = g.n, K = g.k1;
    const int64_t nt = (K + kTK - 1) / kTK;
    const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * kThinWaves + (threadIdx.x >> 6)) *
                       kThinRows;
    const bool active = m0 < M;  // every wave joins the barrier below
    const float* A = g.a1;
    const int64_t lda = g.lda1;

    float a0[2][8], a1[2][8], a2[2][8];
    auto fetch = [&](int64_t kt, float (&ra)[2][8]) {
        const int64_t k = kt * kTK + 8 * q;
        const int64_t kv = K - k;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t gm = m0 + 16 * i + r;
            const float* p = A + (gm < M ? gm : 0) * lda + (kv > 0 ? k : 0);
            if (gm < M && kv >= 8) {
                const Float4Dw x0 = *reinterpret_cast<const Float4Dw*>(p);
                const Float4Dw x1 = *reinterpret_cast<const Float4Dw*>(p + 4);
                ra[i][0] = x0.x; ra[i][1] = x0.y; ra[i][2] = x0.z; ra[i][3] = x0.w;
                ra[i][4] = x1.x; ra[i][5] = x1.y; ra[i][6] = x1.z; ra[i][7] = x1.w;
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) ra[i][t] = (gm < M && t < kv) ? p[t] : 0.0f;
            }
        }
    };
    if (active && nt > 0) fetch(0, a0);
    if (active && nt > 1) fetch(1, a1);
    // stage B, zero-padded to nt * 32 rows and BN columns: eight loads in
    // flight per thread before their stores (a load-store loop waited out
    // one load latency per element)
    const int64_t kp = nt * kTK;
    const int64_t total = kp * BN;
    for (int64_t e0 = threadIdx.x; e0 < total; e0 += 8 * static_cast<int64_t>(blockDim.x)) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t e = e0 + u * static_cast<int64_t>(blockDim.x);
            const int64_t k = e / BN, c = e % BN;
            v[u] = (e < total && k < K && c < N) ? g.b1[k * g.ldb1 + c] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t e = e0 + u * static_cast<int64_t>(blockDim.x);
            const int64_t k = e / BN, c = e % BN;
            if (e < total) Bs[((k >> 3) * BN + c) * 8 + (k & 7)] = v[u];
        }
    }
    __syncthreads();
    if (!active) return;

    v4f acc[2][NT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t kt = 0; kt < nt; ++kt) {
        if (kt + 2 < nt) fetch(kt + 2, a2);
        float b[NT][8];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const float* src = Bs + ((kt * 4 + q) * BN + 16 * j + r) * 8;
            const float4 x0 = *reinterpret_cast<const float4*>(src);
            const float4 x1 = *reinterpret_cast<const float4*>(src + 4);
            b[j][0] = x0.x; b[j][1] = x0.y; b[j][2] = x0.z; b[j][3] = x0.w;
            b[j][4] = x1.x; b[j][5] = x1.y; b[j][6] = x1.z; b[j][7] = x1.w;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[i][s], b[j][s], acc[i][j],
                                                                     0, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                a0[i][t] = a1[i][t];
                a1[i][t] = a2[i][t];
            }
    }
    store_tiles_any(g, acc, m0, 0, q, r);
}

// ---------------------------------------------------------------------------
// Elementwise and row epilogues
// ---------------------------------------------------------------------------
enum { OP_RELU = 0, OP_LEAKY = 1, OP_ELU = 2, OP_SIGMOID = 3, OP_TANH = 4, OP_GELU = 5 };

template <int OP>
__device__ __forceinline__ float unary(float x, float alpha) {
    if constexpr (OP == OP_RELU) return (0.0f < x) ? x : 0.0f;
    if constexpr (OP == OP_LEAKY) return x >= 0.0f ? x : alpha * x;
    if constexpr (OP == OP_ELU) return x < 0.0f ? alpha * (expf(x) - 1.0f) : x;
    if constexpr (OP == OP_SIGMOID) {
        if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
        const float ex = expf(x);
        return ex / (1.0f + ex);
    }
    if constexpr (OP == OP_TANH) return tanhf(x);
    if constexpr (OP == OP_GELU) {
        // (0.5 x)(1 + tanh(c0 (x + c1 x^3))), the cube term fused as the
        // reference build contracts it: fma((c1 x) x, x, x).
        const float inner = 0.7978845608f * __builtin_fmaf((0.044715f * x) * x, x, x);
        return (0.5f * x) * (1.0f + tanhf(inner));
    }
    return x;
}

template <int OP>
__global__ __launch_bounds__(256) void unary_kernel(float* __restrict__ x, int64_t n, float alpha) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        x[i] = unary<OP>(x[i], alpha);
}

__global__ __launch_bounds__(256) void bias_act_kernel(float* __restrict__ x, int64_t rows,
                                                       int64_t cols, int64_t ld,
                                                       const float* __restrict__ bias, int act,
                                                       int post) {
    const int64_t n = rows * cols;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < n;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t i = t / cols, j = t % cols;
        float v = x[i * ld + j];
        if (bias) v = v + bias[j];
        if (act == TG_ACT_RELU) v = (0.0f < v) ? v : 0.0f;
        if (post == TG_POST_RELU) {
            v = (0.0f < v) ? v : 0.0f;
        } else if (post == TG_POST_ELU) {
            if (v < 0.0f) v = 1.0f * (expf(v) - 1.0f);
        }
        x[i * ld + j] = v;
    }
}

// One thread per row; the reference's sequential order (ops.cpp:520-606).
template <bool LOG>
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* __restrict__ x, int64_t rows,
                                                           int64_t cols) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    float* row = x + i * cols;
    float mx = row[0];
    for (int64_t j = 1; j < cols; ++j)
        if (row[j] > mx) mx = row[j];
    float s = 0.0f;
    if constexpr (LOG) {
        for (int64_t j = 0; j < cols; ++j) s += expf(row[j] - mx);
        const float lse = mx + logf(s);
        for (int64_t j = 0; j < cols; ++j) row[j] -= lse;
    } else {
        for (int64_t j = 0; j < cols; ++j) {
            const float e = expf(row[j] - mx);
            row[j] = e;
            s += e;
        }
        const float inv = 1.0f / s;
        for (int64_t j = 0; j < cols; ++j) row[j] *= inv;
    }
}

// edge_softmax (layers.cpp:768-822): one thread per row, sequential.
__global__ __launch_bounds__(256) void edge_softmax_kernel(const int32_t* __restrict__ rp,
                                                           int64_t n,
                                                           const float* __restrict__ v,
                                                           float* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int b = rp[i], e = rp[i + 1];
    if (b == e) return;
    float mx = v[b];
    for (int nz = b + 1; nz < e; ++nz) mx = (mx < v[nz]) ? v[nz] : mx;
    float s = 0.0f;
    for (int nz = b; nz < e; ++nz) {
        const float t = expf(v[nz] - mx);
        out[nz] = t;
        s += t;
    }
    if (s > 0.0f) {
        const float inv = 1.0f / s;
        for (int nz = b; nz < e; ++nz) out[nz] *= inv;
    }
}

unsigned ew_grid(int64_t n) {
    int64_t b = ceil_div(n, 256);
    if (b < 1) b = 1;
    if (b > 16384) b = 16384;
    return static_cast<unsigned>(b);
}

template <int BM, int BN, int TM, int TN, bool DUAL>
void launch_inorder(const GemmArgs& g, hipStream_t s) {
    dim3 grid(static_cast<unsigned>(ceil_div(g.m, BM)), static_cast<unsigned>(ceil_div(g.n, BN)));
    gemm_inorder_kernel<BM, BN, TM, TN, DUAL><<<grid, 256, 0, s>>>(g);
    TG_LAUNCH_CHECK();
}

template <int BN, bool DUAL>
void launch_inorder_small(const GemmArgs& g, hipStream_t s) {
    dim3 grid(static_cast<unsigned>(ceil_div(g.m, 256 / BN)),
              static_cast<unsigned>(ceil_div(g.n, BN)));
    gemm_inorder_small_kernel<BN, DUAL><<<grid, 256, 0, s>>>(g);
    TG_LAUNCH_CHECK();
}

template <int TM, int KT, bool DUAL>
void launch_inorder_rows(const GemmArgs& g, hipStream_t s) {
    dim3 grid(static_cast<unsigned>(ceil_div(g.m, 4 * TM)), static_cast<unsigned>(ceil_div(g.n, 64)));
    gemm_inorder_rows_kernel<TM, KT, DUAL><<<grid, 256, 0, s>>>(g);
    TG_LAUNCH_CHECK();
}

template <bool DUAL>
void dispatch_inorder(const GemmArgs& g, hipStream_t s) {
    // Small products (m n <= 2^21): one output per thread, many workgroups
    // (Cora-scale GCN / SAGE / GAT forwards); the kernels below give such
    // products a few dozen workgroups at most.
    if (g.m * g.n <= (int64_t(1) << 21)) {
        if (g.n <= 8) return launch_inorder_small<8, DUAL>(g, s);
        if (g.n <= 16) return launch_inorder_small<16, DUAL>(g, s);
        if (g.n <= 32) return launch_inorder_small<32, DUAL>(g, s);
        if constexpr (DUAL) return launch_inorder_rows<1, 32, DUAL>(g, s);
        return launch_inorder_small<64, DUAL>(g, s);
    }
    if (g.n > 32) {
        // the 8x8 register-blocked kernel; 128-bit A loads at dword addresses
        auto aligned = [](const float* p, int64_t) {
            return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 3) == 0;
        };
        const bool va4 = aligned(g.a1, g.lda1) && (!DUAL || aligned(g.a2, g.lda2));
        dim3 grid(static_cast<unsigned>(ceil_div(g.m, kWBM)),
                  static_cast<unsigned>(ceil_div(g.n, kWBN)));
        if (va4)
            gemm_inorder_wide_kernel<4, DUAL><<<grid, 256, 0, s>>>(g);
        else
            gemm_inorder_wide_kernel<1, DUAL><<<grid, 256, 0, s>>>(g);
        TG_LAUNCH_CHECK();
        return;
    }
    if (g.n > 16) return launch_inorder<128, 32, 4, 4, DUAL>(g, s);
    if (g.n > 8 || DUAL) return launch_inorder<256, 16, 4, 4, DUAL>(g, s);
    return launch_inorder<256, 8, 4, 2, DUAL>(g, s);
}

void unary_launch(int op, float* x, int64_t n, float alpha, hipStream_t s) {
    if (n <= 0) return;
    require(x != nullptr, "activation: x is null");
    switch (op) {
        case OP_RELU: unary_kernel<OP_RELU><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        case OP_LEAKY: unary_kernel<OP_LEAKY><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        case OP_ELU: unary_kernel<OP_ELU><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        case OP_SIGMOID: unary_kernel<OP_SIGMOID><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        case OP_TANH: unary_kernel<OP_TANH><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        case OP_GELU: unary_kernel<OP_GELU><<<ew_grid(n), 256, 0, s>>>(x, n, alpha); break;
        default: throw std::logic_error("unary op");
    }
    TG_LAUNCH_CHECK();
}

void softmax_launch(bool log, int64_t rows, int64_t cols, float* x, hipStream_t s) {
    const char* fn = log ? "log_softmax_inplace" : "softmax_inplace";
    require(rows >= 0 && cols >= 0, std::string(fn) + ": negative size");
    if (cols == 0)
        throw std::invalid_argument(std::string(fn) + ": tensor has 0 columns — " +
                                    (log ? "log-softmax" : "softmax") +
                                    " over an empty set is undefined.");
    if (rows == 0) return;
    require(x != nullptr, std::string(fn) + ": x is null");
    const unsigned blocks = static_cast<unsigned>(ceil_div(rows, 256));
    if (log)
        softmax_rows_kernel<true><<<blocks, 256, 0, s>>>(x, rows, cols);
    else
        softmax_rows_kernel<false><<<blocks, 256, 0, s>>>(x, rows, cols);
    TG_LAUNCH_CHECK();
}

}  // namespace

int resolve_gemm_algo(int algo, int64_t m, int64_t n, int64_t k) {
    // MFMA only where the product is a real contraction (wide n, deep k and
    // enough work to fill the chip); small products keep the bit-exact
    // in-order kernel.
    // A thin product (n < 64) takes MFMA when A alone is large (m k >= 2^25:
    // config E's n x 256 x 41 layer-2 transforms, 212 us in order); Cora-scale
    // products stay in order.
    if (algo == TG_GEMM_AUTO) {
        if (n >= 64) return (k >= 32 && m * n * k >= (int64_t(1) << 32)) ? TG_GEMM_MFMA
                                                                          : TG_GEMM_INORDER;
        return (k >= 32 && m * k >= (int64_t(1) << 25)) ? TG_GEMM_MFMA : TG_GEMM_INORDER;
    }
    return algo;
}

void gemm(const GemmArgs& g, int algo, hipStream_t s) {
    require(g.m >= 0 && g.n >= 0 && g.k1 >= 0 && g.k2 >= 0, "matmul: negative dimension");
    require(g.epi == TG_EPI_NONE || g.epi == TG_EPI_RELU || g.epi == TG_EPI_ELU,
            "matmul: unknown epilogue");
    require(algo == TG_GEMM_AUTO || algo == TG_GEMM_INORDER || algo == TG_GEMM_MFMA,
            "matmul: unknown algorithm");
    if (g.m == 0 || g.n == 0) return;
    require(g.c != nullptr && (g.c_tile_stride > 0 ? g.ldc == 32 : g.ldc >= g.n),
            "matmul: bad output");
    require(g.c_tile_stride == 0 || g.c_tile_stride >= g.m * 32,
            "matmul: tile-major output stride smaller than a tile");
    require(g.k1 == 0 || (g.a1 && g.b1 && g.lda1 >= g.k1 && g.ldb1 >= g.n),
            "matmul: bad first operand pair");
    const bool dual = g.a2 != nullptr;
    if (dual)
        require(g.b2 && g.lda2 >= g.k2 && g.ldb2 >= g.n, "matmul: bad second operand pair");
    algo = resolve_gemm_algo(algo, g.m, g.n, g.k1 + g.k2);
    if (algo == TG_GEMM_MFMA && g.n <= 64) {
        // thin: one wavefront per 64 rows, 16-column MFMA tiles up to n
        const unsigned grid = static_cast<unsigned>(ceil_div(g.m, 256));
        auto al4 = [](const float* p, int64_t) {  // 128-bit loads at dword addresses
            return p == nullptr || reinterpret_cast<uintptr_t>(p) % 4 == 0;
        };
        const bool aligned = al4(g.a1, g.lda1) && (!dual || al4(g.a2, g.lda2));
        const int ntile = static_cast<int>(ceil_div(g.n, 16));
        const int64_t panel = ceil_div(g.k1, kTK) * kTK * 16 * ntile;  // B floats in LDS
        if (!dual && aligned && panel <= kThinLdsFloats) {
            const unsigned lgrid = static_cast<unsigned>(ceil_div(g.m, kThinRows * kThinWaves));
            const size_t lds = static_cast<size_t>(panel) * sizeof(float);
#define TG_THIN_LDS_CASE(NT_)                                                                      \
            if (ntile == NT_) {                                                                    \
                gemm_mfma_thin_lds_kernel<NT_><<<lgrid, 64 * kThinWaves, lds, s>>>(g);             \
                TG_LAUNCH_CHECK();                                                                 \
                return;                                                                            \
            }
            TG_THIN_LDS_CASE(1) TG_THIN_LDS_CASE(2) TG_THIN_LDS_CASE(3) TG_THIN_LDS_CASE(4)
#undef TG_THIN_LDS_CASE
        }
#define TG_THIN_CASE(NT_)                                                                  \
        if (ntile == NT_) {                                                                \
            if (aligned)                                                                   \
                gemm_mfma_thin_kernel<NT_, true><<<grid, 256, 0, s>>>(g);                  \
            else                                                                           \
                gemm_mfma_thin_kernel<NT_, false><<<grid, 256, 0, s>>>(g);                 \
            TG_LAUNCH_CHECK();                                                             \
            return;                                                                        \
        }
        TG_THIN_CASE(1) TG_THIN_CASE(2) TG_THIN_CASE(3) TG_THIN_CASE(4)
#undef TG_THIN_CASE
    }
    if (algo == TG_GEMM_MFMA) {
        // eight XCDs, each over its row tiles (gemm_mfma_kernel's mapping)
        const int64_t wgs = 8 * ceil_div(ceil_div(g.m, kMBM), 8) * ceil_div(g.n, kMBN);
        require(wgs < (int64_t(1) << 31), "matmul: too many row tiles");
        dim3 grid(static_cast<unsigned>(wgs));
        // 128-bit loads at any dword address (load4)
        auto width = [](std::initializer_list<int64_t>, std::initializer_list<const void*> ps) {
            for (const void* p : ps)
                if (reinterpret_cast<uintptr_t>(p) % sizeof(float) != 0) return 1;
            return 4;
        };
        const int va = dual ? width({g.lda1, g.lda2}, {g.a1, g.a2}) : width({g.lda1}, {g.a1});
        const int vb = dual ? width({g.ldb1, g.ldb2}, {g.b1, g.b2}) : width({g.ldb1}, {g.b1});
#define TG_MFMA_CASE(A_, B_, E_)                                                            \
        if (va == A_ && vb == B_ && g.epi == E_) {                                          \
            gemm_mfma_kernel<A_, B_, E_><<<grid, 256, 0, s>>>(g);                           \
            TG_LAUNCH_CHECK();                                                              \
            return;                                                                         \
        }
#define TG_MFMA_CASES(E_) \
        TG_MFMA_CASE(4, 4, E_) TG_MFMA_CASE(4, 1, E_) TG_MFMA_CASE(1, 4, E_) TG_MFMA_CASE(1, 1, E_)
        TG_MFMA_CASES(TG_EPI_NONE) TG_MFMA_CASES(TG_EPI_RELU) TG_MFMA_CASES(TG_EPI_ELU)
#undef TG_MFMA_CASES
#undef TG_MFMA_CASE
        throw std::logic_error("matmul: no MFMA kernel for this access width");
    }
    if (dual) {
        require(g.k1 == g.k2, "matmul: the in-order dual product needs equal k");
        require(g.tail_from < 0 || g.tail_from % 8 == 0,
                "matmul: the dual product's tail columns must start at a multiple of 8");
        return dispatch_inorder<true>(g, s);
    }
    dispatch_inorder<false>(g, s);
}

void add_bias_act(float* x, int64_t rows, int64_t cols, int64_t ld, const float* bias, int act,
                  int post, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    if (!bias && act == TG_ACT_NONE && post == TG_POST_NONE) return;
    bias_act_kernel<<<ew_grid(rows * cols), 256, 0, s>>>(x, rows, cols, ld, bias, act, post);
    TG_LAUNCH_CHECK();
}

void log_softmax_rows(float* x, int64_t rows, int64_t cols, hipStream_t s) {
    softmax_launch(true, rows, cols, x, s);
}

}  // namespace tg

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
using tg::guard;
using tg::require;

extern "C" {

int tg_matmul(int64_t m, int64_t k, int64_t n, const float* a, int64_t lda, const float* b,
              int64_t ldb, float* c, int64_t ldc, const float* bias, int epilogue, int algo,
              tg_stream_t stream) {
    return guard([&] {
        tg::GemmArgs g;
        g.m = m;
        g.n = n;
        g.k1 = k;
        g.a1 = a;
        g.lda1 = lda;
        g.b1 = b;
        g.ldb1 = ldb;
        g.c = c;
        g.ldc = ldc;
        g.bias = bias;
        g.epi = epilogue;
        tg::gemm(g, algo, static_cast<hipStream_t>(stream));
    });
}

int tg_relu(int64_t n, float* x, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_RELU, x, n, 0.0f, static_cast<hipStream_t>(stream)); });
}
int tg_leaky_relu(int64_t n, float* x, float alpha, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_LEAKY, x, n, alpha, static_cast<hipStream_t>(stream)); });
}
int tg_elu(int64_t n, float* x, float alpha, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_ELU, x, n, alpha, static_cast<hipStream_t>(stream)); });
}
int tg_sigmoid(int64_t n, float* x, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_SIGMOID, x, n, 0.0f, static_cast<hipStream_t>(stream)); });
}
int tg_tanh(int64_t n, float* x, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_TANH, x, n, 0.0f, static_cast<hipStream_t>(stream)); });
}
int tg_gelu(int64_t n, float* x, tg_stream_t stream) {
    return guard([&] { tg::unary_launch(tg::OP_GELU, x, n, 0.0f, static_cast<hipStream_t>(stream)); });
}
int tg_softmax(int64_t rows, int64_t cols, float* x, tg_stream_t stream) {
    return guard([&] { tg::softmax_launch(false, rows, cols, x, static_cast<hipStream_t>(stream)); });
}
int tg_log_softmax(int64_t rows, int64_t cols, float* x, tg_stream_t stream) {
    return guard([&] { tg::softmax_launch(true, rows, cols, x, static_cast<hipStream_t>(stream)); });
}
int tg_add_bias(int64_t rows, int64_t cols, float* x, const float* bias, tg_stream_t stream) {
    return guard([&] {
        require(rows >= 0 && cols >= 0, "add_bias: negative size");
        require(rows * cols == 0 || (x && bias), "add_bias: null pointer");
        tg::add_bias_act(x, rows, cols, cols, bias, TG_ACT_NONE, TG_POST_NONE,
                         static_cast<hipStream_t>(stream));
    });
}

int tg_edge_softmax(int64_t n_rows, const int32_t* row_ptr, const float* val, float* val_out,
                    tg_stream_t stream) {
    return guard([&] {
        require(n_rows >= 0, "edge_softmax: negative size");
        if (n_rows == 0) return;
        require(row_ptr && val && val_out, "edge_softmax: null pointer");
        tg::edge_softmax_kernel<<<static_cast<unsigned>(tg::ceil_div(n_rows, 256)), 256, 0,
                                  static_cast<hipStream_t>(stream)>>>(row_ptr, n_rows, val,
                                                                       val_out);
        TG_LAUNCH_CHECK();
    });
}

}  // extern "C"
