/*
 * tinygnn_amd.h -- C-ABI of the MI355X (gfx950) TinyGNN sparse-inference path.
 *
 * This is the drop-in boundary: plain C, POD arguments, device pointers,
 * int64 sizes, an int status, and a HIP stream passed as `tg_stream_t`
 * (a hipStream_t; NULL = the default stream).  No exception crosses it.
 *
 * Each entry point names the reference interface it replaces
 * (AnubhavChoudhery/TinyGNN, path:line).  Layout conventions match the
 * reference `Tensor` (include/tinygnn/tensor.hpp:14-93): dense matrices are
 * row-major fp32 with a leading dimension (ld >= cols); CSR matrices are
 * row_ptr int32[rows+1], col_ind int32[nnz], val fp32[nnz].
 *
 * Status codes map onto the exceptions the reference throws:
 *   TG_ERR_INVALID_ARGUMENT -> std::invalid_argument (format/shape errors)
 *   TG_ERR_RUNTIME          -> std::runtime_error    (I/O, empty Model)
 *   TG_ERR_OUT_OF_RANGE     -> std::out_of_range
 * and tg_last_error() returns the message (thread-local, reference text).
 *
 * Unless stated otherwise calls are asynchronous on `stream`; inputs must
 * stay valid until the stream reaches the call.  Entry points that must
 * report a data-dependent error the reference raises (edge_list_to_csr's
 * endpoint check, CSR validation) synchronise the stream, and say so.
 */
#ifndef TINYGNN_AMD_H
#define TINYGNN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tg_stream_t; /* hipStream_t */

enum {
    TG_OK = 0,
    TG_ERR_INVALID_ARGUMENT = 1,
    TG_ERR_RUNTIME = 2,
    TG_ERR_OUT_OF_RANGE = 3,
    TG_ERR_HIP = 4,
    TG_ERR_ALLOC = 5
};

/* Activation applied by a layer (layers.hpp:Activation {None=0, ReLU=1}). */
enum { TG_ACT_NONE = 0, TG_ACT_RELU = 1 };
/* Post-layer activation (model.hpp:92-96 InterActivation {None, ReLU, ELU}). */
enum { TG_POST_NONE = 0, TG_POST_RELU = 1, TG_POST_ELU = 2 };
/* SAGE aggregator (layers.hpp:250-253 {Mean=0, Max=1}). */
enum { TG_AGG_MEAN = 0, TG_AGG_MAX = 1 };
/* Epilogue fused into a matmul or SpMM store: bias add, then ReLU or ELU
 * (alpha 1), as add_bias then relu_inplace / elu_inplace (ops.cpp:328-661). */
enum { TG_EPI_NONE = 0, TG_EPI_RELU = 1, TG_EPI_ELU = 2 };
/* Summation order of SpMM plans and Model forwards (no counterpart in the
 * reference, which has one order): TG_PRECISION_EXACT keeps the reference's
 * order bit for bit; TG_PRECISION_FAST may regroup sums (see the entry
 * points that take it). */
enum { TG_PRECISION_FAST = 0, TG_PRECISION_EXACT = 1 };

/* Message of the last failed call on this thread ("" if none). */
const char* tg_last_error(void);

/* Library version, (major << 16) | minor. */
int tg_version(void);

/* ------------------------------------------------------------------------
 * CSR construction -- replaces GraphLoader::edge_list_to_csr
 * (src/graph_loader.cpp:211-281, include/tinygnn/graph_loader.hpp:74-76).
 * Row = source.  Output is bit-identical to the reference: out-degree
 * row_ptr, each row's destinations sorted ascending with duplicates kept,
 * values 1.0f.  row_ptr has n_nodes+1 entries, col_ind/val n_edges.
 * Endpoints outside [0, n_nodes) fail with TG_ERR_INVALID_ARGUMENT naming
 * the first bad edge (this check synchronises `stream`).
 * `workspace` may be NULL (the library then allocates and frees it).
 * ------------------------------------------------------------------------ */
size_t tg_edge_list_to_csr_workspace_size(int64_t n_nodes, int64_t n_edges);
int tg_edge_list_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src,
                        const int32_t* dst, int32_t* row_ptr, int32_t* col_ind,
                        float* val, void* workspace, size_t workspace_bytes,
                        tg_stream_t stream);

/* ------------------------------------------------------------------------
 * CSR validation -- replaces the checks of Tensor::sparse_csr
 * (src/tensor.cpp:41-96): col_ind within [0, n_cols), row_ptr
 * non-decreasing, row_ptr[n_rows] == nnz.  Synchronises `stream`.
 * ------------------------------------------------------------------------ */
/* The CSR that the pybind module's Tensor.from_edge_index and
 * load_cora_binary build (python/tinygnn_ext.cpp:116-157, src/model.cpp:
 * 87-126): rows = sources, destinations sorted, duplicates kept, values
 * 1.0f, and destinations checked only afterwards, by Tensor::sparse_csr's
 * validation (an out-of-range one raises "Tensor::sparse_csr: col_ind[k] =
 * v is out of bounds for cols=n" at its sorted position).  A source outside
 * [0, n_nodes) -- undefined behaviour in the reference -- raises
 * TG_ERR_INVALID_ARGUMENT "<context>: edge[k].src = v out of range [0, n)".
 * Synchronises. */
int tg_coo_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src, const int32_t* dst,
                  int32_t* row_ptr, int32_t* col_ind, float* val, const char* context,
                  tg_stream_t stream);
int tg_csr_validate(int64_t n_rows, int64_t n_cols, int64_t nnz,
                    const int32_t* row_ptr, const int32_t* col_ind,
                    tg_stream_t stream);

/* ------------------------------------------------------------------------
 * Self-loops and symmetric normalisation -- replace add_self_loops
 * (src/layers.cpp:71-144) and gcn_norm (src/layers.cpp:158-208).
 * A must be square (n x n).  Outputs need capacity nnz + n; the produced
 * nnz' = row_ptr_out[n] (= nnz + number of rows without a diagonal).
 * Structure, values, degrees and 1/sqrt(deg) are bit-identical to the
 * reference.  deg_out / dis_out (length n) may be NULL.
 * ------------------------------------------------------------------------ */
size_t tg_self_loops_workspace_size(int64_t n);
int tg_add_self_loops(int64_t n, int64_t nnz, const int32_t* row_ptr,
                      const int32_t* col_ind, const float* val,
                      int32_t* row_ptr_out, int32_t* col_ind_out, float* val_out,
                      void* workspace, size_t workspace_bytes, tg_stream_t stream);
int tg_gcn_norm(int64_t n, int64_t nnz, const int32_t* row_ptr,
                const int32_t* col_ind, const float* val, int32_t* row_ptr_out,
                int32_t* col_ind_out, float* val_out, float* deg_out,
                float* dis_out, void* workspace, size_t workspace_bytes,
                tg_stream_t stream);

/* ------------------------------------------------------------------------
 * CSR SpMM -- replaces tinygnn::spmm (src/ops.cpp:198-297, ops.hpp:112):
 * C[m x f] = A[m x k] * B[k x f].
 *
 * A plan holds the degree-binned row schedule of one CSR structure
 * (row_ptr): rows of at most `chunk_nnz` nonzeros (0 = default, 1,024) are
 * chunks of their own, ordered longest first, each summed by one lane per
 * output element with fma in nonzero order -- the reference's chain, bit
 * for bit.  Longer rows ("split rows", listed longest first) are summed,
 * by default (TG_PRECISION_EXACT), as the same single chain, one workgroup
 * per row: the whole output is bit-identical to the reference.  Under
 * TG_PRECISION_FAST they are cut into chunks whose per-chunk partials are
 * added in chunk order (deterministic, a regrouped sum).  `nnz_bound` >=
 * the actual nnz (row_ptr[m]); `max_f` bounds the feature width of later
 * executes.  Plan creation allocates device memory and synchronises
 * `stream` once.
 * ------------------------------------------------------------------------ */
typedef struct tg_spmm_plan_s* tg_spmm_plan_t;
int tg_spmm_plan_create(int64_t m, int64_t nnz_bound, const int32_t* row_ptr,
                        int64_t max_f, int64_t chunk_nnz, tg_stream_t stream,
                        tg_spmm_plan_t* plan_out);
int tg_spmm_plan_destroy(tg_spmm_plan_t plan);
/* Number of chunks and of multi-chunk rows (diagnostics). */
int tg_spmm_plan_info(tg_spmm_plan_t plan, int64_t* n_chunks, int64_t* n_split_rows,
                      int64_t* n_partials);
int tg_spmm_execute(tg_spmm_plan_t plan, int64_t k, int64_t f,
                    const int32_t* row_ptr, const int32_t* col_ind, const float* val,
                    const float* b, int64_t ldb, float* c, int64_t ldc,
                    tg_stream_t stream);
/* tg_spmm_execute with the epilogue of GCNLayer::forward fused into the
 * store (src/layers.cpp:319-336): C = act(A B + bias), bias of f floats (or
 * NULL), epilogue TG_EPI_NONE / TG_EPI_RELU / TG_EPI_ELU (alpha 1).  The
 * result is bit-identical to tg_spmm_execute, then tg_add_bias, then
 * tg_relu / tg_elu, without the two extra passes over C. */
int tg_spmm_execute_epilogue(tg_spmm_plan_t plan, int64_t k, int64_t f,
                             const int32_t* row_ptr, const int32_t* col_ind,
                             const float* val, const float* b, int64_t ldb, float* c,
                             int64_t ldc, const float* bias, int epilogue,
                             tg_stream_t stream);
/* Summation order of the plan's later executes and of tg_sage_aggregate /
 * tg_sage_forward over it (TG_PRECISION_EXACT by default).  EXACT sums
 * every row, split rows included, as one chain in nonzero order from 0 --
 * the reference's order (src/ops.cpp:252-294) -- so the whole output is
 * bit-identical to the reference: a row longer than the plan's chunk runs
 * on one workgroup, its gathers spread over the workgroup, its chains
 * walked in order from LDS.  FAST: split rows from per-chunk partials. */
int tg_spmm_plan_set_precision(tg_spmm_plan_t plan, int precision);
/* One-shot form: builds a plan, executes, frees it (allocates; synchronises).
 * tg_spmm is tg_spmm_ex with TG_PRECISION_EXACT (bit-identical). */
int tg_spmm_ex(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
               const int32_t* col_ind, const float* val, const float* b, int64_t ldb,
               float* c, int64_t ldc, int precision, tg_stream_t stream);
int tg_spmm(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
            const int32_t* col_ind, const float* val, const float* b, int64_t ldb,
            float* c, int64_t ldc, tg_stream_t stream);

/* ------------------------------------------------------------------------
 * SpMM that allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Arguments and
 * result bits are tg_spmm's (the same plan and kernels: every row in the
 * reference's order), but the plan lives in a fixed device array of
 * TG_SPMM_NOALLOC_SCRATCH_BYTES per GPU, and the call neither allocates nor
 * synchronises: it only enqueues kernels on `stream`.
 *   The array is the only content of its code object, which a GPU loads
 *   when a process first calls tg_spmm_noalloc on it (resolving the array's
 *   address): from then until the process ends, that GPU holds the 128 MiB
 *   for that process; processes that never call it do not hold it.  That
 *   first call on each GPU must be made outside stream capture (under
 *   capture it fails with TG_ERR_INVALID_ARGUMENT); later calls may be
 *   captured into HIP graphs and replayed.
 *   Limit: the plan takes 16(m+1) + 16(m + nnz/1024) + 16 nnz/1025
 *   + 4 round_up(f, 4) (nnz/1024 + nnz/1025) bytes, about (256-byte aligned
 *   pieces); larger sizes fail with TG_ERR_INVALID_ARGUMENT before any device
 *   work.  Config D (10^6 rows, 5 x 10^7 nonzeros) fits for f <= 256.
 *   Every call on one GPU uses that GPU's one array and leaves its contents
 *   behind: calls that overlap in time on one GPU (other streams, other
 *   threads, graph replays) race, and the caller must serialise them.
 *   row_ptr[m] must equal nnz, as for tg_spmm; a larger row_ptr[m] that
 *   overflows the plan's capacities fills C with NaN.
 * ------------------------------------------------------------------------ */
#define TG_SPMM_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int tg_spmm_noalloc(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
                    const int32_t* col_ind, const float* val, const float* b, int64_t ldb,
                    float* c, int64_t ldc, tg_stream_t stream);

/* ------------------------------------------------------------------------
 * Dense transform -- replaces tinygnn::matmul (src/ops.cpp:70-162,
 * ops.hpp:76): C[m x n] = A[m x k] * B[k x n], with an optional fused
 * epilogue (bias add, then activation) that equals calling add_bias
 * (ops.cpp:622) and relu_inplace / elu_inplace afterwards.
 * algo: TG_GEMM_AUTO picks fp32 MFMA when n >= 64, k >= 32 and
 * m*n*k >= 2^32, else the in-order kernel; TG_GEMM_INORDER is bit-identical
 * to the reference (one fma chain over k ascending from 0 per output);
 * TG_GEMM_MFMA uses v_mfma_f32_16x16x4f32 (regrouped sums: within
 * tolerance, not bit-identical).
 * ------------------------------------------------------------------------ */
enum { TG_GEMM_AUTO = 0, TG_GEMM_INORDER = 1, TG_GEMM_MFMA = 2 };
int tg_matmul(int64_t m, int64_t k, int64_t n, const float* a, int64_t lda,
              const float* b, int64_t ldb, float* c, int64_t ldc,
              const float* bias, int epilogue, int algo, tg_stream_t stream);

/* ------------------------------------------------------------------------
 * Epilogues -- replace the in-place activations and add_bias
 * (src/ops.cpp:328-661).  Dense row-major, contiguous.
 * ------------------------------------------------------------------------ */
int tg_relu(int64_t n, float* x, tg_stream_t stream);
int tg_leaky_relu(int64_t n, float* x, float alpha, tg_stream_t stream);
int tg_elu(int64_t n, float* x, float alpha, tg_stream_t stream);
int tg_sigmoid(int64_t n, float* x, tg_stream_t stream);
int tg_tanh(int64_t n, float* x, tg_stream_t stream);
int tg_gelu(int64_t n, float* x, tg_stream_t stream);
int tg_softmax(int64_t rows, int64_t cols, float* x, tg_stream_t stream);
int tg_log_softmax(int64_t rows, int64_t cols, float* x, tg_stream_t stream);
int tg_add_bias(int64_t rows, int64_t cols, float* x, const float* bias,
                tg_stream_t stream);

/* ------------------------------------------------------------------------
 * edge_softmax -- replaces tinygnn::edge_softmax (src/layers.cpp:768-822):
 * row softmax over the CSR values; structure unchanged; empty rows kept.
 * ------------------------------------------------------------------------ */
int tg_edge_softmax(int64_t n_rows, const int32_t* row_ptr, const float* val,
                    float* val_out, tg_stream_t stream);

/* ------------------------------------------------------------------------
 * GraphSAGE -- replaces SAGELayer::forward (src/layers.cpp:538-752) and
 * sage_max_aggregate (src/layers.cpp:359-435).
 * tg_sage_aggregate writes AGG[n x f]: the mean (sum in nonzero order,
 * times 1.0f/deg; edge values ignored; duplicates counted) or the
 * element-wise max (0 for rows without neighbours).  Uses `plan` for A.
 * tg_sage_forward computes out = act(AGG*Wn + H*Ws + b):
 *   dataflow TG_SAGE_CONCAT aggregates H at f_in, then one GEMM over the
 *     concatenation [AGG | H] against [Wn ; Ws]  (needs workspace for AGG);
 *   dataflow TG_SAGE_TRANSFORM_FIRST computes T = H*[Ws | Wn] first and
 *     aggregates T's neighbour half at f_out (mean only; fewer bytes);
 *   TG_SAGE_AUTO takes transform-first for the mean aggregator when
 *     f_out < f_in and nnz * f_in >= 2^26, else concat.
 * With concat and the in-order GEMM (small products) the result is
 * bit-identical to the reference (every row under a plan of
 * TG_PRECISION_EXACT, the default; rows of at most one chunk under FAST).
 * `nnz` of the workspace query is the adjacency's nonzero count.
 * ------------------------------------------------------------------------ */
enum { TG_SAGE_AUTO = 0, TG_SAGE_CONCAT = 1, TG_SAGE_TRANSFORM_FIRST = 2 };
int tg_sage_aggregate(tg_spmm_plan_t plan, int64_t n, int64_t f, int agg,
                      const int32_t* row_ptr, const int32_t* col_ind,
                      const float* h, int64_t ldh, float* out, int64_t ldo,
                      tg_stream_t stream);
size_t tg_sage_forward_workspace_size(int64_t n, int64_t f_in, int64_t f_out,
                                      int agg, int dataflow, int64_t nnz);
int tg_sage_forward(tg_spmm_plan_t plan, int64_t n, int64_t f_in, int64_t f_out,
                    int agg, const int32_t* row_ptr, const int32_t* col_ind,
                    const float* h, const float* w_neigh, const float* w_self,
                    const float* bias, int act, int post, int dataflow,
                    float* out, void* workspace, size_t workspace_bytes,
                    tg_stream_t stream);

/* ------------------------------------------------------------------------
 * GAT, all heads of one layer at once -- replaces GATLayer::forward
 * (src/layers.cpp:945-1129) run per head plus Model's head concat/average
 * (src/model.cpp:312-354, :403-421).
 * wh: [n x heads*f] (head-major columns, ld = ldwh), the transformed
 * features of every head.  att_l / att_r / bias: [heads x f].
 * tg_gat_scores: src[i*heads+h] = a_l(h).Wh_i(h), dst likewise with a_r, in
 * the reference's operation order (layers.cpp:991-1026).
 * tg_gat_aggregate: per row i and head h, e_ij = LeakyReLU(src_i + dst_j),
 * softmax over the row, out_i(h) = sum alpha_ij Wh_j(h) + b(h), then the
 * layer activation `act` and the model's post activation `post`; heads are
 * concatenated (out is [n x heads*f]) or averaged (concat = 0, [n x f]).
 * The nnz x heads attention matrix is never stored.  `plan` is the plan of
 * A + I's structure (values are not read); its max_f must be >= heads*f
 * when it has split rows.  The workspace (size from
 * tg_gat_workspace_size; NULL = allocated by the call) holds per-chunk
 * softmax statistics of split rows and, when heads are averaged, the
 * per-head outputs.
 * ------------------------------------------------------------------------ */
int tg_gat_scores(int64_t n, int64_t heads, int64_t f, const float* wh,
                  int64_t ldwh, const float* att_l, const float* att_r, float* src,
                  float* dst, tg_stream_t stream);
size_t tg_gat_workspace_size(tg_spmm_plan_t plan, int64_t n, int64_t heads,
                             int64_t f, int concat);
int tg_gat_aggregate(tg_spmm_plan_t plan, int64_t n, int64_t heads, int64_t f,
                     const int32_t* row_ptr, const int32_t* col_ind, const float* wh,
                     int64_t ldwh, const float* src, const float* dst, float slope,
                     const float* bias, int act, int post, int concat, float* out,
                     int64_t ldo, void* workspace, size_t workspace_bytes,
                     tg_stream_t stream);

/* ------------------------------------------------------------------------
 * Model -- replaces tinygnn::Model (include/tinygnn/model.hpp:89-164,
 * src/model.cpp:191-439): a sequential GCN / SAGE / GAT layer graph with
 * device-resident weights.
 *   tg_model_add_*_layer  <- Model::add_{gcn,sage,gat}_layer (:191-247)
 *   tg_model_set_tensor   <- one WeightFile entry (model.hpp:76-79);
 *                            host data, copied.  Names as model.hpp:131-135.
 *   tg_model_load_weights <- Model::load_weights(const WeightFile&) (:258-305)
 *   tg_model_forward      <- Model::forward (:359-439).  adjacency: raw CSR
 *     (no self-loops) on the device; x: [n x f_in] device features; out:
 *     [n x out_cols] device.  mode TG_FORWARD_REFERENCE recomputes gcn_norm /
 *     add_self_loops on every call as the reference does (src/model.cpp:
 *     373-381); TG_FORWARD_CACHED reuses them (and the SpMM plans and
 *     blocked copies) while the adjacency pointers, sizes, the precision and
 *     the layer list are unchanged.  The cache cannot see the adjacency's
 *     contents: a caller that edits row_ptr / col_ind / val in place, or
 *     frees them and passes new arrays that may land at the same addresses,
 *     must call tg_model_invalidate first (or pass TG_FORWARD_REFERENCE,
 *     which also refreshes the cache).  The C++ API (tinygnn::Model) and the
 *     Python front end do this from the tensors' versions.  The model owns
 *     its intermediate buffers.
 *   tg_model_invalidate   forgets the cached adjacency state (no counterpart
 *     in the reference, which keeps none); the next forward recomputes it.
 * ------------------------------------------------------------------------ */
typedef struct tg_model_s* tg_model_t;
enum { TG_FORWARD_REFERENCE = 0, TG_FORWARD_CACHED = 1 };
int tg_model_create(tg_model_t* model_out);
int tg_model_destroy(tg_model_t model);
int tg_model_add_gcn_layer(tg_model_t model, int64_t in_f, int64_t out_f, int bias,
                           int act, int post, int64_t* index_out);
int tg_model_add_sage_layer(tg_model_t model, int64_t in_f, int64_t out_f, int agg,
                            int bias, int act, int post, int64_t* index_out);
int tg_model_add_gat_layer(tg_model_t model, int64_t in_f, int64_t out_f,
                           int64_t heads, int concat, float neg_slope, int bias,
                           int act, int post, int64_t* index_out);
int tg_model_num_layers(tg_model_t model, int64_t* n_out);
int tg_model_output_cols(tg_model_t model, int64_t* cols_out);
int tg_model_set_tensor(tg_model_t model, const char* name, int64_t rows,
                        int64_t cols, const float* host_data);
/* Forgets every staged tensor (a new WeightFile replaces the old one). */
int tg_model_clear_tensors(tg_model_t model);
int tg_model_load_weights(tg_model_t model);
/* SAGE dataflow used by the model's SAGE-mean layers (TG_SAGE_*). */
int tg_model_set_sage_dataflow(tg_model_t model, int dataflow);
/* Precision of the model's forward:
 *   TG_PRECISION_FAST (default): fp32 MFMA for the wide transforms, rows of
 *     more than one plan chunk summed from per-chunk partials, SAGE
 *     transform-first on large graphs, GAT with a one-pass online softmax;
 *     within 1e-4 relative / 1e-5 absolute of the reference.
 *   TG_PRECISION_EXACT: the reference's operation order everywhere -- in-order
 *     GEMMs, every row one fma chain (no row splitting), SAGE concat, GAT's
 *     max / sequential sum / alpha = t*(1/sum) per row with exp and ELU
 *     evaluated in double and rounded.  GCN and SAGE outputs are
 *     bit-identical to the reference; GAT differs only where the reference's
 *     libm expf is not correctly rounded. */
int tg_model_set_precision(tg_model_t model, int precision);
/* Column blocking of the model's GCN, SAGE-mean and GAT aggregations
 * (both forward modes; GAT layers with concatenated or single heads of
 * whole 32-column tiles; in exact precision only for adjacencies whose rows
 * are in column order, where the blocked sums keep the reference's order
 * bit for bit; no counterpart in the reference, which has one CPU loop per
 * row).  rows_per_block > 0 cuts the adjacency's columns into blocks of
 * that many source nodes (at least n/64) and aggregates block by block, so
 * each pass gathers from a slice of the feature matrix that stays in L2;
 * 0 disables it; -1 (the default) uses equal blocks of at most 23552 rows for
 * weighted passes over A + I (GAT, and GCN in exact precision or on
 * weighted graphs: 64-column lane groups) and 38912 rows for passes without
 * values (SAGE mean over A; fast GCN over an A + I whose values are all 1:
 * 32-column groups) when the graph holds at least 8 entries per row and
 * block.  The blocked copy of the adjacency is built with the other
 * preprocessing of the forward (one more copy of col_ind, and of val for
 * weighted passes). */
int tg_model_set_blocking(tg_model_t model, int64_t rows_per_block);
int tg_model_forward(tg_model_t model, int64_t n, int64_t nnz,
                     const int32_t* row_ptr, const int32_t* col_ind, const float* val,
                     int64_t f_in, const float* x, float* out, int mode,
                     tg_stream_t stream);
int tg_model_invalidate(tg_model_t model);
/* The column blocking of the cached adjacency state (diagnostics; no
 * counterpart in the reference): blocks and columns per lane group of A + I's
 * blocked copy (GCN, GAT) and of A's (SAGE mean); 0 blocks = unblocked or no
 * cached state; sl_direct = 1 when A + I's blocked copy was split from A
 * directly (below); resident: bit 0 set when A + I's blocked copy is
 * prepared for the output-resident passes, bit 1 when A's is
 * (tg_model_set_resident_passes).  Filled by the last forward; any pointer
 * may be null. */
int tg_model_blocking_info(tg_model_t model, int64_t* blocks_sl, int64_t* cols_sl,
                           int64_t* blocks_raw, int64_t* cols_raw, int64_t* sl_direct,
                           int64_t* resident);
/* How a fast-precision model whose blocked A + I is read only by the
 * factored GCN passes (A's values all 1) or by GAT passes that carry their
 * softmax gets that copy (no counterpart in the reference; for tests and
 * measurement).  direct = 1 (the default): when A's rows are sorted and
 * without a diagonal, the blocked copy is split from A directly, each row's
 * diagonal placed where add_self_loops would insert it (and, for GCN,
 * gcn_norm's degrees come from the row lengths); A + I itself is never
 * written.  The build checks those conditions and otherwise takes the path
 * of direct = 0: gcn_norm / add_self_loops write A + I's structure, which is
 * then split.  Both give the same blocked copy and the same outputs bit for
 * bit.  Drops the cached state. */
int tg_model_set_self_loop_split(tg_model_t model, int direct);
/* The blocked aggregations without values in fast precision (SAGE mean;
 * the factored GCN over a unit A + I) as output-resident passes (no
 * counterpart in the reference; for tests and measurement).  on = 1: one
 * workgroup per CU owns a range of rows (at most 1088; used when the rows
 * fit, n <= 1088 x CUs) and keeps their 32-column output tile in LDS while
 * it walks every column block, each block's entries of the range split
 * evenly over its lane groups; one launch per aggregation, the output
 * written once, the workgroups paced block by block so that they gather
 * from one block's slice of B at a time.  on = 0 (the default): one pass
 * per block, each reading and writing the output (config E: the resident
 * form reaches a 94% L2 hit rate but keeps fewer gathers in flight, and is
 * slower).  The sums are deterministic either way and differ in rounding
 * only.  Drops the cached state. */
int tg_model_set_resident_passes(tg_model_t model, int on);

/* ------------------------------------------------------------------------
 * CSV ingestion -- replaces GraphLoader::parse_edges / parse_features and
 * the reading half of GraphLoader::load (src/graph_loader.cpp:61-206,
 * 286-326).  The text is indexed into lines once on the device (lines split
 * at '\n', trimmed of " \t\r\n", empty ones dropped: read_lines, :38-53;
 * line 0 is a header when a letter or '_' precedes its first ',', ' ' or
 * '\t': is_header, :24-33), then parsed as an edge list or a feature table.
 * Fields convert with std::stoi / std::stof semantics (glibc strtol /
 * strtof, bit for bit, ERANGE included).  Errors are std::runtime_error
 * (TG_ERR_RUNTIME) with the reference's messages, for the first failing line
 * in file order; line numbers count the non-empty lines from 1.
 *   tg_csv_open           reads a file into device memory and indexes it
 *                         ("GraphLoader: cannot open file '<path>'").
 *   tg_csv_index          indexes text already in device memory; the text
 *                         must outlive the handle.  name is used in messages.
 *   tg_csv_parse_edges    <- parse_edges (:61-107): one (src, dst) per data
 *                         line into device int32 src[], dst[] of
 *                         n_lines - has_header entries; max_id_out (host,
 *                         optional) receives the largest endpoint, -1 if none.
 *   tg_csv_feature_shape  <- parse_features' dimensions (:118-183): rows =
 *                         largest node_id + 1, cols = the first data line's
 *                         feature count.  Reports only "file is empty" /
 *                         "no data rows"; field errors come from the parse.
 *   tg_csv_parse_features <- parse_features (:112-206): out (device,
 *                         n_rows >= rows, leading dimension ld >= cols) gets
 *                         in row r the features of the last line whose
 *                         node_id is r, zeros where no line has that node_id,
 *                         and zeros in rows [rows, n_rows) (the zero padding
 *                         of GraphLoader::load, :311-320).
 * All of them synchronise the stream (data-dependent sizes and errors).
 * ------------------------------------------------------------------------ */
typedef struct tg_csv_s* tg_csv_t;
int tg_csv_open(const char* path, tg_csv_t* csv_out, tg_stream_t stream);
int tg_csv_index(const char* text, int64_t n_bytes, const char* name, tg_csv_t* csv_out,
                 tg_stream_t stream);
int tg_csv_destroy(tg_csv_t csv);
int tg_csv_info(tg_csv_t csv, int64_t* n_lines, int* has_header);
int tg_csv_parse_edges(tg_csv_t csv, int32_t* src, int32_t* dst, int64_t* max_id_out,
                       tg_stream_t stream);
int tg_csv_feature_shape(tg_csv_t csv, int64_t* rows, int64_t* cols, tg_stream_t stream);
int tg_csv_parse_features(tg_csv_t csv, float* out, int64_t n_rows, int64_t ld,
                          tg_stream_t stream);

/* ------------------------------------------------------------------------
 * TGNN weight file, version 1 -- replaces load_weight_file
 * (src/model.cpp:134-185; format include/tinygnn/model.hpp:22-33).  Read on
 * the host; entries keep the file's order (a repeated name: the last one is
 * what the reference's map keeps).  Errors are std::runtime_error with the
 * reference's messages ("load_weight_file: cannot open <path>", "... invalid
 * magic in <path>", "... unsupported version <v> in <path>", "...: unexpected
 * end of file or read error.").  tg_weights_tensor's pointers are host
 * memory owned by the handle.  Model::load_weights(path) is tg_weights_open,
 * tg_model_set_tensor per entry, tg_model_load_weights.
 * ------------------------------------------------------------------------ */
typedef struct tg_weights_s* tg_weights_t;
int tg_weights_open(const char* path, tg_weights_t* out);
int tg_weights_info(tg_weights_t w, int64_t* n_tensors, float* test_accuracy);
int tg_weights_tensor(tg_weights_t w, int64_t i, const char** name, int64_t* name_len,
                      int64_t* rows, int64_t* cols, const float** data);
int tg_weights_destroy(tg_weights_t w);

/* ------------------------------------------------------------------------
 * Cora binary export -- replaces load_cora_binary (src/model.cpp:49-129).
 * tg_cora_open reads the file on the host (errors as the reference:
 * "load_cora_binary: cannot open <path>", "load_cora_binary: unexpected end
 * of file or read error.").  tg_cora_upload copies the features to the
 * device ([num_nodes x num_features]) and builds the adjacency there
 * (row_ptr[num_nodes + 1], col_ind / val[num_edges]): rows = sources,
 * destinations sorted, duplicates kept, values 1.0f, then the checks of
 * Tensor::sparse_csr (an out-of-range destination raises
 * "Tensor::sparse_csr: col_ind[k] = ..." at its sorted position, as in the
 * reference).  A source outside [0, num_nodes), undefined behaviour in the
 * reference, raises std::invalid_argument.  tg_cora_host's arrays are host
 * memory owned by the handle.
 * ------------------------------------------------------------------------ */
typedef struct tg_cora_s* tg_cora_t;
int tg_cora_open(const char* path, tg_cora_t* out);
int tg_cora_info(tg_cora_t c, int64_t* num_nodes, int64_t* num_features,
                 int64_t* num_classes, int64_t* num_edges);
int tg_cora_host(tg_cora_t c, const int32_t** labels, const uint8_t** train_mask,
                 const uint8_t** val_mask, const uint8_t** test_mask);
int tg_cora_upload(tg_cora_t c, float* features, int32_t* row_ptr, int32_t* col_ind,
                   float* val, tg_stream_t stream);
int tg_cora_destroy(tg_cora_t c);

/* ------------------------------------------------------------------------
 * Measurement (no counterpart in the reference): the L2 read ceiling.
 * Each of `workgroups` 256-thread workgroups reads the whole of `buf`
 * (`bytes`, a power of two >= 32 KB, 16-byte aligned; a few MB stay in each
 * XCD's 4 MB L2) with 16-byte loads; sink receives workgroups x 256 floats.
 * Bytes read = workgroups x bytes.  Asynchronous on `stream`.
 * ------------------------------------------------------------------------ */
int tg_probe_l2_read(const void* buf, int64_t bytes, int64_t workgroups, float* sink,
                     tg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TINYGNN_AMD_H */
