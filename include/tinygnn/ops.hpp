// tinygnn/ops.hpp -- compute kernels of TinyGNN's API (reference
// include/tinygnn/ops.hpp:76-286), running on the MI355X through the C-ABI
// in tinygnn_amd.h.  Same names, arguments, results and exceptions.
#pragma once

#include <cstddef>

#include "tinygnn/tensor.hpp"

namespace tinygnn {

/// C = A * B, both Dense (ops.cpp:70-162).  Small products are bit-identical
/// to the reference; wide ones (n >= 64, k >= 32, m*n*k >= 2^32) run on fp32
/// MFMA (within 1e-4 relative).
Tensor matmul(const Tensor& A, const Tensor& B);

/// C = A * B, A SparseCSR, B Dense (ops.cpp:198-297).  Every row is one
/// fma chain in nonzero order, as in the reference: bit-identical.
Tensor spmm(const Tensor& A, const Tensor& B);

/// Summation order of spmm (an addition of this build: the reference has
/// one order).  Exact is the reference's and spmm(A, B)'s; Fast sums rows
/// longer than 1,024 nonzeros from per-chunk partials (a regrouped sum,
/// within the fp32 summation bound of the exact one).
enum class SpmmOrder : uint8_t { Exact = 0, Fast = 1 };
Tensor spmm(const Tensor& A, const Tensor& B, SpmmOrder order);

void relu_inplace(Tensor& X);
void leaky_relu_inplace(Tensor& X, float alpha = 0.01f);
void elu_inplace(Tensor& X, float alpha = 1.0f);
void sigmoid_inplace(Tensor& X);
void tanh_inplace(Tensor& X);
void gelu_inplace(Tensor& X);
void softmax_inplace(Tensor& X);
void log_softmax_inplace(Tensor& X);
void add_bias(Tensor& X, const Tensor& bias);

}  // namespace tinygnn
