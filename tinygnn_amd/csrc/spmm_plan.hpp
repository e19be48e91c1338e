// spmm_plan.hpp -- the row schedule shared by every CSR aggregation kernel
// (SpMM, SAGE aggregation, GAT aggregation).
//
// A plan cuts every row of a CSR structure into chunks of at most
// `chunk` nonzeros (an empty row is one empty chunk, so it still writes its
// zero output), and lists the chunks longest first in 64 length bins (two
// per octave).  One lane group processes one chunk; consecutive groups
// therefore get chunks of similar length.  A row of more than one chunk
// ("split row") gets one partial-result slot per chunk; a second kernel
// adds its partials in chunk order, so results are deterministic.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

struct tg_spmm_plan_s {
    int64_t m = 0;
    int64_t nnz_bound = 0;
    int64_t max_f = 0;
    int64_t chunk = 0;
    int64_t n_chunks = 0;
    int64_t n_split = 0;
    int64_t n_partials = 0;
    int device = 0;
    // summation order of the plan's executes: TG_PRECISION_EXACT (the
    // default) sums split rows as single in-order chains, TG_PRECISION_FAST
    // from per-chunk partials
    int precision = TG_PRECISION_EXACT;
    const int32_t* row_ptr = nullptr;   // the structure the plan was built for
    tg::DeviceBuffer chunks;            // int4 {row, begin, end, slot (-1 = direct)}
    tg::DeviceBuffer split;             // int4 {row, first slot, n chunks, degree}
    tg::DeviceBuffer partials;          // float [n_partials x max_f]
    tg::DeviceBuffer scratch;           // the build's temporaries (kept for rebuilds)
    tg::PinnedBuffer host_totals;       // the count phase's totals, read by the host
};

namespace tg {

// A plan's arrays as the aggregation launches read them.  For an owning
// plan the counts are exact and dev_counts is null.  For a plan built into
// tg_spmm_noalloc's static scratch the host never learns the counts:
// n_chunks / n_split are upper bounds (they size the grids) and
// dev_counts[0] / dev_counts[1] hold the true counts in device memory, read
// by the kernels (workgroups past them exit).
struct PlanView {
    int64_t m = 0;
    int64_t max_f = 0;
    int64_t n_chunks = 0;
    int64_t n_split = 0;
    const int4* chunks = nullptr;
    const int4* split = nullptr;
    float* partials = nullptr;
    const int64_t* dev_counts = nullptr;
    const int32_t* row_ptr = nullptr;  // the structure's row pointers (split rows' starts)
};

inline PlanView plan_view(const tg_spmm_plan_s& p) {
    PlanView v;
    v.m = p.m;
    v.max_f = p.max_f;
    v.n_chunks = p.n_chunks;
    v.n_split = p.n_split;
    v.chunks = p.chunks.as<int4>();
    v.split = p.split.as<int4>();
    v.partials = p.partials.as<float>();
    v.row_ptr = p.row_ptr;
    return v;
}

constexpr int kPlanBins = 64;
constexpr int64_t kDefaultChunk = 1024;

// Builds the plan (synchronises `s` once, for the chunk count).  Buffers only
// grow: rebuilding a plan object for a structure of the same size allocates
// nothing.
void build_plan(tg_spmm_plan_s& p, int64_t m, int64_t nnz_bound, const int32_t* row_ptr,
                int64_t max_f, int64_t chunk, hipStream_t s);

// The same build in two phases, so that several plans share one
// synchronisation: build_plan_count enqueues the counting and the copy of
// the three totals to host_totals (pinned host memory, 3 int64); once `s`
// has synchronised, build_plan_finish sizes the plan and enqueues the
// scatter.
void build_plan_count(tg_spmm_plan_s& p, int64_t m, int64_t nnz_bound, const int32_t* row_ptr,
                      int64_t max_f, int64_t chunk, hipStream_t s, int64_t* host_totals);
void build_plan_finish(tg_spmm_plan_s& p, const int64_t* host_totals, hipStream_t s);

// nplans (<= kMaxMultiPlans) plans, plan b over rows [b*m, (b+1)*m) of one
// row-pointer array of nplans*m + 1 absolute offsets (a column-blocked
// copy's block row pointers), built together: one launch per step for all
// plans and one synchronisation of `s`.  Plan b is the plan build_plan
// would make over row_ptr + b*m.  scratch holds the temporaries (it only
// grows); host_totals is pinned host memory of 4*nplans int64.  Work
// enqueued on `s` before the call is complete when it returns.
constexpr int kMaxMultiPlans = 64;
void build_plans_multi(tg_spmm_plan_s* const* plans, int nplans, int64_t m, int64_t nnz_bound,
                       const int32_t* row_ptr, int64_t max_f, int64_t chunk,
                       DeviceBuffer& scratch, int64_t* host_totals, hipStream_t s);

// Lane layout for an aggregation of width f: each lane owns VPL (= 1)
// vectors of VEC consecutive floats, LPR lanes own one row's feature tile,
// and n_tiles tiles cover f.
struct LaneLayout {
    int vec;     // 1, 2 or 4 floats per access
    int lpr;     // lanes per row group: 4, 8, 16, 32 or 64
    int vpl;     // vectors per lane: 1, 2 or 4
    int tile;    // features covered by one group (lpr * vpl * vec)
    int n_tiles; // feature tiles per row
};

LaneLayout choose_layout(int64_t f, int vec);

// Largest access width (4, 2, 1) allowed by f, the leading dimensions and
// the alignment of the pointers.
int pick_vec(int64_t f, std::initializer_list<int64_t> lds,
             std::initializer_list<const void*> ptrs);

// Largest width for loading rows of f valid floats from a matrix of leading
// dimension ldb: the last vector of a row may run into the row's padding
// (round_up(f, v) <= ldb), whose values are loaded and never stored.
int pick_load_vec(int64_t f, int64_t ldb, const void* b);

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// tg_spmm's plan and aggregation with every buffer carved from `scratch`, a
// device array of scratch_bytes (>= spmm_noalloc_bytes(m, nnz, f)): only
// kernels are enqueued on s, nothing is allocated and the host reads no
// count.  C's bits are tg_spmm's; a row_ptr[m] larger than nnz fills C with
// NaN.
size_t spmm_noalloc_bytes(int64_t m, int64_t nnz, int64_t f);
void spmm_noalloc(char* scratch, size_t scratch_bytes, int64_t m, int64_t f, int64_t nnz,
                  const int32_t* rp, const int32_t* ci, const float* v, const float* b,
                  int64_t ldb, float* c, int64_t ldc, hipStream_t s);

// Row pitch (floats) for a dense matrix whose rows are gathered: widths of
// 4, 8, 16 or 32 floats after 4-float padding tile a 128-byte cache line
// exactly; wider rows are padded to whole lines, so a gathered row always
// touches ceil(f / 32) lines and never one more.
inline int64_t gather_pitch(int64_t f) {
    const int64_t p = round_up(f, 4);
    if (p == 4 || p == 8 || p == 16 || p == 32) return p;
    return round_up(f, 32);
}

}  // namespace tg
