// dense.hpp -- dense transforms and epilogues shared by the layers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tg {

// C[m x n] = epi( A1[m x k1] * B1[k1 x n]  (+ A2[m x k2] * B2[k2 x n]) )
// Row-major operands with leading dimensions.  epi: bias add (if bias),
// then TG_EPI_NONE / TG_EPI_RELU / TG_EPI_ELU (alpha 1).
//
// In-order algorithm (TG_GEMM_INORDER): every output is one fma chain over k
// ascending from 0 -- bit-identical to the reference matmul (ops.cpp:120-159).
// With a second pair (k2 == k1), the chain interleaves the pairs per k:
// c = fma(a1, b1, c); c = fma(a2, b2, c) -- the fused SAGE dual matmul
// (layers.cpp:643-659) -- and columns >= tail_from use the reference's
// scalar tail c = c + fma(a1, b1, a2 * b2) (layers.cpp:660-662).
//
// MFMA algorithm (TG_GEMM_MFMA): v_mfma_f32_16x16x4f32 tiles; the pairs are
// concatenated along k.  Not bit-identical (the k order is regrouped).
struct GemmArgs {
    int64_t m = 0, n = 0;
    const float* a1 = nullptr;
    int64_t lda1 = 0;
    const float* b1 = nullptr;
    int64_t ldb1 = 0;
    int64_t k1 = 0;
    const float* a2 = nullptr;
    int64_t lda2 = 0;
    const float* b2 = nullptr;
    int64_t ldb2 = 0;
    int64_t k2 = 0;
    float* c = nullptr;
    int64_t ldc = 0;
    const float* bias = nullptr;
    int epi = 0;
    // per-row factor: C[m, :] = epilogue(row_scale[m] * (A B)[m, :]) (null: none)
    const float* row_scale = nullptr;
    int64_t tail_from = -1;  // in-order dual only; -1 = no tail columns, else a multiple of 8
    // C's layout: 0 = row-major (ldc); > 0 = tile-major, column n of row m at
    // c[(n / 32) * c_tile_stride + m * 32 + n % 32] (ldc = 32): the layout the
    // column-blocked aggregations gather from
    int64_t c_tile_stride = 0;
};

// Resolves TG_GEMM_AUTO: MFMA when n >= 64 and k >= 32, else in order.
int resolve_gemm_algo(int algo, int64_t m, int64_t n, int64_t k);
void gemm(const GemmArgs& g, int algo, hipStream_t s);

// Epilogue helpers (contiguous row-major).
void add_bias_act(float* x, int64_t rows, int64_t cols, int64_t ld, const float* bias, int act,
                  int post, hipStream_t s);
void log_softmax_rows(float* x, int64_t rows, int64_t cols, hipStream_t s);

}  // namespace tg
