// layers.hpp -- library-internal entry points of the graph, SAGE and GAT
// modules, used by the C-ABI wrappers and by the Model.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "spmm_plan.hpp"

namespace tg {

struct BlockedCSR;

// graph.hip
// check_dst = false leaves destinations unchecked (load_cora_binary's build,
// whose result Tensor::sparse_csr validates instead).
// who names the caller in messages (default "GraphLoader::edge_list_to_csr").
void edge_list_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src, const int32_t* dst,
                      int32_t* row_ptr, int32_t* col_ind, float* val, void* workspace,
                      size_t ws_bytes, hipStream_t s, bool check_dst = true,
                      const char* who = nullptr);
size_t edge_list_to_csr_ws(int64_t n_nodes);
void csr_validate(int64_t n_rows, int64_t n_cols, int64_t nnz, const int32_t* row_ptr,
                  const int32_t* col_ind, hipStream_t s);
// values = false: the structure of A + I alone (row_ptr_out, col_out; val_out
// is ignored), and for gcn_norm deg_out / dis_out.
void add_self_loops(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
                    const float* val, int32_t* row_ptr_out, int32_t* col_out, float* val_out,
                    void* ws, size_t ws_bytes, hipStream_t s, bool values = true);
void gcn_norm(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
              const float* val, int32_t* row_ptr_out, int32_t* col_out, float* val_out,
              float* deg_out, float* dis_out, void* ws, size_t ws_bytes, hipStream_t s,
              bool values = true);
size_t self_loops_workspace(int64_t n);
// gcn_norm's dis_out for an A (n x n) whose values are all 1 and which has
// no diagonal, from the row lengths alone (bit-identical to gcn_norm's);
// sets *flag (not cleared) when a row of A + I is longer than 2^24, where
// gcn_norm's result differs.
void unit_self_loop_dis(int64_t n, const int32_t* row_ptr, float* dis, int32_t* flag,
                        hipStream_t s);

// sage.hip
// `blocked` (optional): the column-blocked form of the same structure; the
// mean aggregation then runs block by block (run_aggregate_blocked).
void sage_aggregate(const tg_spmm_plan_s& p, int64_t f, int agg, const int32_t* ci,
                    const float* h, int64_t ldh, float* out, int64_t ldo, hipStream_t s,
                    const BlockedCSR* blocked = nullptr);
size_t sage_forward_ws(int64_t n, int64_t f_in, int64_t f_out, int agg, int dataflow,
                       int64_t nnz);
// t_pre (transform-first only, optional): T = H * [Ws | 0 | Wn | 0]
// already computed by sage_transform with the same `tiled` layout the call
// picks (sage_tf_tiled); the call then starts at the aggregation.
void sage_forward(const tg_spmm_plan_s& p, int64_t n, int64_t f_in, int64_t f_out, int agg,
                  const int32_t* ci, const float* h, const float* wn, const float* ws,
                  const float* bias, int act, int post, int dataflow, float* out, void* work,
                  size_t work_bytes, hipStream_t s, int gemm_algo = TG_GEMM_AUTO,
                  const BlockedCSR* blocked = nullptr, const float* t_pre = nullptr);
// The resolved dataflow (TG_SAGE_AUTO decided as sage_forward does).
int sage_dataflow_for(int dataflow, int agg, int64_t f_in, int64_t f_out, int64_t nnz);
// Transform-first: whether T is stored tile-major (a blocked aggregation
// over 32-column tiles), and T's size in floats.
bool sage_tf_tiled(int64_t f_out, bool blocked);
int64_t sage_tf_floats(int64_t n, int64_t f_out);
// T = H * [Ws | 0 | Wn | 0] into t (sage_tf_floats(n, f_out) floats), with
// wcat (f_in x 2 gather_pitch(f_out) floats) as the concatenated weights.
void sage_transform(int64_t n, int64_t f_in, int64_t f_out, const float* h, const float* wn,
                    const float* ws, bool tiled, float* t, float* wcat, hipStream_t s,
                    int gemm_algo);

// gat.hip
void gat_scores(int64_t n, int64_t heads, int64_t f, const float* wh, int64_t ldwh,
                const float* al, const float* ar, float* src, float* dst, hipStream_t s);
size_t gat_workspace(const tg_spmm_plan_s& p, int64_t n, int64_t heads, int64_t f, int concat);
// The workspace of a blocked GAT aggregation in fast precision (the
// softmax carried across the passes), sized by the block plans.
size_t gat_workspace_blocked(const BlockedCSR& bk, int64_t n, int64_t heads, int64_t f,
                             int concat);
int64_t gat_stat_slots(int64_t heads, int64_t f);
void gat_aggregate(const tg_spmm_plan_s& p, int64_t n, int64_t heads, int64_t f,
                   const int32_t* ci, const float* wh, int64_t ldwh, const float* src,
                   const float* dst, float slope, const float* bias, int act, int post,
                   int concat, float* out, int64_t ldo, void* work, size_t work_bytes,
                   hipStream_t s, bool exact = false);
// Column-blocked GAT aggregation: whether a layer's layout
// allows it (concatenated or single head, heads of whole 32-column tiles),
// and the aggregation itself over the blocked
// form of the structure (plan, ci: the unblocked structure's plan and
// columns, for the softmax statistics of the exact path and of layers whose
// heads are not whole lane groups; null where fast precision carries the
// softmax across the passes; rmax, rinv: n x max(heads, ceil(heads*f/32))
// scratch, the row statistics or, in fast precision, the softmax state the
// passes carry per (row, column group); the passes compute each entry's
// attention weight and store none; work: at least gat_workspace(*plan, ...),
// or gat_workspace_blocked(bk, ...) without a plan
// bytes; exact: the reference's
// operation order, for a plan that splits no row and a blocked structure in
// block order; ar: the attention vector a_r [heads x f] behind dst, or null:
// fast-precision passes whose lane groups hold whole heads then compute
// a_r . Wh_j from the gathered rows instead of reading dst).
bool gat_blocked_ok(int64_t heads, int64_t f, int concat);
void gat_aggregate_blocked(const BlockedCSR& bk, const tg_spmm_plan_s* plan, int64_t n,
                           int64_t heads, int64_t f, const int32_t* ci, const float* wh,
                           int64_t ldwh, const float* src, const float* dst, float slope,
                           const float* bias, int act, int post, float* out, int64_t ldo,
                           float* rmax, float* rinv, void* work, size_t work_bytes,
                           hipStream_t s, bool exact = false, const float* ar = nullptr);

}  // namespace tg
