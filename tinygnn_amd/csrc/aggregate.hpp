// aggregate.hpp -- the chunked CSR aggregation engine (SpMM, SAGE mean,
// GCN propagation) built on a tg_spmm_plan_s.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "spmm_plan.hpp"

namespace tg {

// Applied to a finished output row element, in this order:
//   x *= 1/deg (mean; deg = row length, skipped for deg == 0)
//   x += self[row, :]       (if self)
//   x += bias[:]            (if bias)
//   x  = act(x)             (TG_ACT_NONE / TG_ACT_RELU)
//   x  = post(x)            (TG_POST_NONE / TG_POST_RELU / TG_POST_ELU, alpha 1)
struct AggEpilogue {
    const float* bias = nullptr;
    const float* self = nullptr;
    int64_t ld_self = 0;
    int mean = 0;
    int max = 0;   // element-wise max instead of a sum (SAGE-Max); empty rows give 0
    int act = 0;
    int post = 0;
    int vec_io = 1;  // set by run_aggregate: stores and epilogue loads are full vectors
};

// out[row, :] = epilogue( sum over row nonzeros of w * B[col, :] ), where w is
// val[nz] (fma, in nonzero order) or, when val is null, 1 (plain add); with
// epi.max the element-wise maximum of B[col, :] over the row instead.
void run_aggregate(const tg_spmm_plan_s& plan, int64_t f, const int32_t* col_ind,
                   const float* val, const float* b, int64_t ldb, float* c, int64_t ldc,
                   const AggEpilogue& epi, hipStream_t s);

}  // namespace tg
