// aggregate.hpp -- the chunked CSR aggregation engine (SpMM, SAGE mean,
// GCN propagation) built on a tg_spmm_plan_s.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <vector>

#include "spmm_plan.hpp"

namespace tg {

// Applied to a finished output row element, in this order:
//   x  = out[row, :] + x   (if acc, for rows split into several chunks: a
//                           column-block pass after the first; an unsplit
//                           row's pass starts its sum from out[row, :])
//   x *= 1/deg (mean; deg = row length, or deg_rp's when given; skipped for
//               deg == 0)
//   x *= row_scale[row * scale_ld + col / scale_cols]   (if row_scale)
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
    const int32_t* deg_rp = nullptr;  // mean: degrees from this row_ptr (the unblocked rows)
    int acc = 0;         // add the row's previous value in out
    int skip_empty = 0;  // rows with no entries in this pass keep their value in out
    const float* row_scale = nullptr;  // per row and column group (GAT: 1/sum per head)
    int64_t scale_ld = 0;
    int scale_cols = 1;
    int exact_exp = 0;  // ELU's exp evaluated as exp_rn (the exact GAT path)
    // plain sums (no values, not max or attention): a chunk's last, partial
    // batch gathers nothing for the slots past its end (worth it for the
    // fast blocked passes' chunks, not for long unsplit ones)
    int mask_tail = 0;
    // rows of more than one plan chunk ("split rows") summed as one chain in
    // nonzero order, one workgroup per row (agg_long_kernel), instead of from
    // per-chunk partials: every row then sums in the reference's order
    int long_rows = 0;
    // B's layout (tile_cols = 32 only): > 0 = tile-major, 32-column tile t
    // of row j at B + t * b_tile_stride + j * ldb (ldb = 32); 0 = row-major
    int64_t b_tile_stride = 0;
    // rows of B from its (offset) first row to its end (a blocked pass: the
    // rows from the block's first source row), set only where every 16-bit
    // column is below 65535; 0 = unknown.  Lets the 16-bit passes gather
    // through buffer loads that read zeros past the end.
    int64_t b_rows = 0;
    // self's layout: > 0 = tile-major as B (ld_self = 32); 0 = row-major
    int64_t self_tile_stride = 0;
    // columns per head of the attention mode below (tiles never straddle
    // two heads)
    int w_head_cols = 1;
    // 16-bit column indices (a blocked pass): used instead of col_ind, as
    // offsets from B's (and att_dst's) first row, which the caller offsets to
    // the block's first source row
    const uint16_t* ci16 = nullptr;
    // GAT attention computed in the pass (att_dst non-null): the weight of
    // entry (i, j) for the tile's head h = first column / w_head_cols is
    // exp(LeakyReLU(att_src[i,h] + att_dst[j,h]) - att_max[i,h]) *
    // att_rinv[i,h], with exact_exp choosing exp_rn; all four arrays are
    // [n x att_heads].  No value stream is read.
    const float* att_src = nullptr;
    const float* att_dst = nullptr;
    const float* att_max = nullptr;
    const float* att_rinv = nullptr;
    int att_heads = 1;
    float att_slope = 0.2f;
};


// out[row, :] = epilogue( sum over row nonzeros of w * B[col, :] ), where w is
// val[nz] (fma, in nonzero order) or, when val is null, 1 (plain add); with
// epi.max the element-wise maximum of B[col, :] over the row instead.
//
// tile_cols = 0 picks the lane layout from f.  tile_cols = 32 or 64 makes
// every lane group cover one column group of that many floats (one or two
// 128-byte lines per gathered row; with a tile-major B the two lines come
// from two adjacent tiles), groups running in grid order, so the workgroups
// resident at a time gather from the rows of one or two groups (the
// column-blocked passes size their blocks for that).
void run_aggregate(const tg_spmm_plan_s& plan, int64_t f, const int32_t* col_ind,
                   const float* val, const float* b, int64_t ldb, float* c, int64_t ldc,
                   const AggEpilogue& epi, hipStream_t s, int tile_cols = 0);
// The same over a plan view (a plan in fixed scratch, counts on the device).
void run_aggregate(const PlanView& plan, int64_t f, const int32_t* col_ind, const float* val,
                   const float* b, int64_t ldb, float* c, int64_t ldc, const AggEpilogue& epi,
                   hipStream_t s, int tile_cols = 0);

// Column-blocked form of a CSR structure for aggregations whose gathered
// matrix is larger than an XCD's L2: the columns (source nodes) are cut into
// blocks of `rows_per_block`, and each block's nonzeros form a CSR of their
// own ([block][row] order, the row's order kept inside a block), with one
// row plan per block.  An aggregation then runs one pass per block, so the
// lines of B it gathers in a pass (rows_per_block x 128 bytes per 32-column
// tile) stay in L2; passes add into out in block order (deterministic).
struct BlockedCSR {
    int64_t n = 0, nnz = 0, rows_per_block = 0, n_blocks = 0;
    // columns per lane group in the passes (32 or 64, see resolve_block_rows)
    int group_cols = 32;
    const int32_t* rp = nullptr;  // row_ptr of the source structure (full row degrees)
    bool weighted = false;
    // every row's entries fall in non-decreasing blocks (e.g. sorted
    // columns): block order is nonzero order, so unsplit rows (plans built
    // with chunk >= the longest row) sum in the unblocked order bit for bit
    bool in_order = false;
    // set by the caller before the build: also prepare the output-resident
    // passes (run_aggregate_resident) for the copy's plain sums, where the
    // indices are 16-bit and the rows fit the workgroups' LDS
    bool resident = false;
    // the resident passes' row ranges, one per workgroup (0 = not prepared):
    // int32 [resident_wgs + 1] first rows, balanced by entries
    int64_t resident_wgs = 0;
    DeviceBuffer wg_rows;
    // the resident passes' phase counters (one per column tile and block,
    // for the tiles of max_f columns), cleared before each launch
    DeviceBuffer phase_count;
    int64_t max_phases = 0;
    // the copy holds A + I's entries with rp = A's row_ptr (each row's
    // diagonal placed by the split, build_blocked_self_loops)
    bool vdiag = false;
    DeviceBuffer brp;  // int32 [n_blocks * n + 1]
    // the entries' columns: with idx16 (blocks of at most 65,536 rows) uint16
    // offsets within their block, column - block * rows_per_block (half the
    // index stream of a pass: config-E forwards 2.5-3% faster); else int32
    bool idx16 = false;
    DeviceBuffer bci;
    DeviceBuffer bv;   // float [nnz] (weighted structures)
    DeviceBuffer scratch;       // the build's temporaries
    DeviceBuffer plan_scratch;  // the block plans' build temporaries
    PinnedBuffer host;          // the build's device-to-host results (plan totals, disorder)
    std::vector<std::unique_ptr<tg_spmm_plan_s>> plans;
    // called once by the next build, right after it enqueues the copy's
    // scatter (before the block plans), then cleared: a caller starts other
    // streams' work there, so that it does not take the CUs from the split's
    // latency-bound passes
    std::function<void()> after_split;
};

// Blocks with at most 64 column blocks; v may be null (structure only);
// chunk: the per-block plans' chunk size (0 = default).  Rebuilding into the
// same object reuses its buffers and plans (they only grow).  Synchronises
// `s` (once when every row is sorted, twice otherwise).
void build_blocked(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                   const int32_t* ci, const float* v, int64_t rows_per_block, int64_t max_f,
                   hipStream_t s, int64_t chunk = 0);

// The blocked copy of A + I's structure (nnz + n entries, no values) built
// from A's (n x n, nnz entries) directly, each row's diagonal entry placed
// before its first column > i, as add_self_loops inserts it: valid when
// every row of A is sorted and none has a diagonal.  Returns false when
// that does not hold (the copy is then unusable); bk.rp is A's row_ptr.
bool build_blocked_self_loops(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                              const int32_t* ci, int64_t rows_per_block, int64_t max_f,
                              hipStream_t s, int64_t chunk = 0);

// Rows per block for an n-node structure with nnz entries whose passes use
// lane groups of group_cols columns: `requested` > 0 is taken as given, 0
// disables blocking, < 0 picks the default (equal blocks of at most 38912
// rows for 32-column groups, 23552 for 64-column ones: 4.75 / 5.75 MB of the
// gathered lines) when the passes pay for their extra output traffic (a
// mean of at least 8 entries per row and block).  Returns 0 when the
// structure should not be blocked.
int64_t resolve_block_rows(int64_t requested, int64_t n, int64_t nnz, int group_cols = 32);

// The same aggregation as run_aggregate over the unblocked structure (same
// epilogue; weights from the blocked values when bk is weighted, or computed
// per entry in the attention mode), computed block by block, each pass
// continuing the rows' sums.  With bk.in_order and plans that split no row,
// the result is bit-identical to the unblocked in-order sums; rows split
// into chunks are summed from per-chunk partials.  epi.max is not supported.
void run_aggregate_blocked(const BlockedCSR& bk, int64_t f, const float* b, int64_t ldb,
                           float* c, int64_t ldc, const AggEpilogue& epi, hipStream_t s);

// The output-resident passes (fast precision; plain sums over 16-bit
// indices): one workgroup per CU owns a range of at most kResidentRows rows
// and keeps their 32-column output tile in LDS while it walks every column
// block in order, so all workgroups gather from one block's slice of B at a
// time (the slice stays in L2) and no pass reads or writes the output in
// between.  Each block's entries of the range are split evenly over the
// workgroup's lane groups; a row cut by such a split is summed as the
// owning group's chain plus the later groups' partials, in group order
// (deterministic; the unblocked and the per-pass sums differ in rounding
// only).  Requires bk.resident_wgs > 0, and B with 16-byte aligned rows
// (tile-major, or row-major with ldb % 4 == 0).
constexpr int kResidentThreads = 1024;  // per workgroup
constexpr int kResidentPerCU = 1;       // workgroups per CU (LDS: 157 KB)
constexpr int kResidentRows = 1088;
bool resident_ok(const BlockedCSR& bk, int64_t f, const float* b, int64_t ldb,
                 const AggEpilogue& epi);
void run_aggregate_resident(const BlockedCSR& bk, int64_t f, const float* b, int64_t ldb,
                            float* c, int64_t ldc, const AggEpilogue& epi, hipStream_t s);
// Splits bk's rows into bk.resident_wgs ranges (one per CU, at most
// kResidentRows rows each, balanced by entries) and sizes the phase
// counters for widths up to max_f; leaves resident_wgs = 0 when the rows do
// not fit.  No synchronisation.
void build_resident_split(BlockedCSR& bk, int64_t max_f, hipStream_t s);

}  // namespace tg
