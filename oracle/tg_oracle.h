/*
 * tg_oracle.h -- CPU restatement of TinyGNN's sparse-inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path
 * is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never
 * links, calls or falls back to it.
 *
 * Every function restates the algorithm of the reference file:line quoted
 * beside it (paths relative to the reference repository root), with the
 * same loop order and the same floating-point operation sequence: each
 * fused multiply-add of the reference (AVX2 _mm256_fmadd_ps lanes and the
 * scalar tails that GCC contracts under its default -ffp-contract=fast) is
 * an explicit fmaf() here, and this file is compiled with
 * -ffp-contract=off so no other operation is fused.
 *
 * Buffers are caller-allocated; dense matrices are row-major with the
 * leading dimension equal to the column count.  Return value 0 = ok,
 * nonzero = the reference would have thrown (message via or_last_error()).
 */
#ifndef TG_ORACLE_H
#define TG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* or_last_error(void);

/* graph_loader.cpp:211-281 -- count, scan, scatter in input order, per-row
 * sort, values 1.0f. */
int or_edge_list_to_csr(int64_t n_nodes, int64_t n_edges,
                        const int32_t* src, const int32_t* dst,
                        int32_t* row_ptr, int32_t* col_ind, float* val);

/* layers.cpp:83-93 -- number of nonzeros of A + I. */
int64_t or_add_self_loops_nnz(int64_t n, const int32_t* rp, const int32_t* ci);

/* layers.cpp:71-144 -- A + I in sorted position. */
void or_add_self_loops(int64_t n, const int32_t* rp, const int32_t* ci,
                       const float* v, int32_t* rp_out, int32_t* ci_out,
                       float* v_out);

/* layers.cpp:158-208 -- D^-1/2 (A+I) D^-1/2.  deg_out / dis_out (length n)
 * may be NULL; they receive the degree and inverse square root arrays. */
void or_gcn_norm(int64_t n, const int32_t* rp, const int32_t* ci,
                 const float* v, int32_t* rp_out, int32_t* ci_out,
                 float* v_out, float* deg_out, float* dis_out);

/* ops.cpp:198-297 -- C[M x F] = A_csr[M x K] * B[K x F]. */
void or_spmm(int64_t m, int64_t f, const int32_t* rp, const int32_t* ci,
             const float* av, const float* b, float* c);
/* checker: float64 products of selected rows and their sums of |terms| */
void or_spmm_rows_f64(int64_t n_sel, const int32_t* rows, int64_t f, const int32_t* rp,
                      const int32_t* ci, const float* av, const float* b, double* exact,
                      double* absum);

/* ops.cpp:70-162 -- C[M x N] = A[M x K] * B[K x N], (i,k,j) order. */
void or_matmul(int64_t m, int64_t k, int64_t n, const float* a,
               const float* b, float* c);

/* ops.cpp:328-392, 411-546, 565-661 -- in-place epilogues. */
void or_relu(int64_t n, float* x);
void or_leaky_relu(int64_t n, float* x, float alpha);
void or_elu(int64_t n, float* x, float alpha);
void or_sigmoid(int64_t n, float* x);
void or_tanh(int64_t n, float* x);
void or_gelu(int64_t n, float* x);
void or_softmax(int64_t m, int64_t n, float* x);
void or_log_softmax(int64_t m, int64_t n, float* x);
void or_add_bias(int64_t m, int64_t n, float* x, const float* bias);

/* layers.cpp:768-822 -- row softmax over CSR values (structure unchanged). */
void or_edge_softmax(int64_t n, const int32_t* rp, const float* v,
                     float* v_out);

/* layers.cpp:359-435 -- element-wise neighbour max (0 for empty rows). */
void or_sage_max_aggregate(int64_t n, int64_t f, const int32_t* rp,
                           const int32_t* ci, const float* h, float* out);

/* layers.cpp:538-752 -- fused SAGE forward.  agg: 0 = Mean, 1 = Max.
 * act: 0 = None, 1 = ReLU.  bias may be NULL when use_bias == 0. */
void or_sage_forward(int64_t n, int64_t f_in, int64_t f_out, int agg,
                     const int32_t* rp, const int32_t* ci, const float* h,
                     const float* w_neigh, const float* w_self,
                     const float* bias, int use_bias, int act, float* out);

/* layers.cpp:286-339 -- GCN forward on a pre-normalised adjacency. */
void or_gcn_forward(int64_t n, int64_t f_in, int64_t f_out,
                    const int32_t* rp, const int32_t* ci, const float* av,
                    const float* h, const float* w, const float* bias,
                    int use_bias, int act, float* out);

/* layers.cpp:991-1026 -- per-node attention dots (src = a_l, dst = a_r). */
void or_gat_scores(int64_t n, int64_t f, const float* wh, const float* al,
                   const float* ar, float* src, float* dst);

/* layers.cpp:945-1129 -- single-head GAT forward on A with self-loops.
 * wh_out (n x f_out, may be NULL) receives H*W. */
void or_gat_forward(int64_t n, int64_t f_in, int64_t f_out,
                    const int32_t* rp, const int32_t* ci, const float* h,
                    const float* w, const float* al, const float* ar,
                    const float* bias, float slope, int use_bias, int act,
                    float* out);

/* graph_loader.cpp:61-107 -- GraphLoader::parse_edges over an in-memory
 * text (name is used in messages).  Writes up to cap edges; *n_out receives
 * the count.  Returns 2 (std::runtime_error) on the reference's errors. */
int or_parse_edges(const char* text, int64_t n, const char* name, int32_t* src,
                   int32_t* dst, int64_t cap, int64_t* n_out);

/* graph_loader.cpp:112-206 -- GraphLoader::parse_features over an
 * in-memory text.  *rows_out x *cols_out is the table's shape; out is
 * written when it holds at least that many floats (else only the shape). */
int or_parse_features(const char* text, int64_t n, const char* name, float* out,
                      int64_t cap, int64_t* rows_out, int64_t* cols_out);

/* OpenMP thread count for the parallel loops (<= 0 keeps the default). */
void or_set_num_threads(int n);
int or_get_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
