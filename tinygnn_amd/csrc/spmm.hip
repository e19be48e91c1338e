// spmm.hip -- CSR SpMM for gfx950 and the row-schedule plan it runs on.
//
// Replaces tinygnn::spmm (reference src/ops.cpp:198-297).  The reference
// walks each row's nonzeros in order and does C[i,j] = fma(val, B[col,j],
// C[i,j]) for every feature j.  Here one lane owns VEC consecutive features
// of one row and performs exactly that fma chain, so a row handled as one
// chunk reproduces the reference bit for bit.  What changes is the mapping:
// rows are cut into bounded chunks, binned by length (longest first), and
// LPR lanes (4..64) of a wavefront cover one chunk's feature tile, so a
// wavefront works on 64/LPR rows of similar length at once and issues
// U independent 128-bit gathers of B rows per lane before consuming them.
#include "aggregate.hpp"
#include "common.hpp"
#include "device_utils.hpp"
#include "spmm_plan.hpp"

#include <algorithm>
#include <climits>
#include <memory>

namespace tg {

// ---------------------------------------------------------------------------
// Plan construction
// ---------------------------------------------------------------------------
namespace {

// Length bin, two per octave, larger bin = longer chunk.
__device__ __forceinline__ int chunk_bin(int len) {
    if (len <= 1) return len;  // 0 -> 0, 1 -> 1
    int lg = 31 - __clz(len);  // floor(log2 len) >= 1
    int half = (len >> (lg - 1)) & 1;  // second half of the octave
    int b = 2 * lg + half;
    return b < kPlanBins ? b : kPlanBins - 1;
}

// bin_count holds 2 x kPlanBins counters: the chunks' length bins, then the
// split rows' degree bins (split rows are listed longest first too).
__global__ __launch_bounds__(256) void plan_count_kernel(const int32_t* __restrict__ row_ptr,
                                                         int64_t m, int chunk,
                                                         int32_t* __restrict__ split_cnt,
                                                         int32_t* __restrict__ is_split,
                                                         int32_t* __restrict__ bin_count) {
    __shared__ int32_t hist[2 * kPlanBins];
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < m) {
        const int deg = row_ptr[r + 1] - row_ptr[r];
        const int nch = deg <= chunk ? 1 : (deg + chunk - 1) / chunk;
        split_cnt[r] = nch > 1 ? nch : 0;
        is_split[r] = nch > 1 ? 1 : 0;
        if (nch == 1) {
            atomicAdd(&hist[chunk_bin(deg)], 1);
        } else {
            const int full = deg / chunk, rem = deg - full * chunk;
            atomicAdd(&hist[chunk_bin(chunk)], full);
            if (rem) atomicAdd(&hist[chunk_bin(rem)], 1);
            atomicAdd(&hist[kPlanBins + chunk_bin(deg)], 1);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x)
        if (hist[i]) atomicAdd(&bin_count[i], hist[i]);
}

// Turns bin counts into start cursors, longest bin first; writes totals.
// With caps (a plan built into fixed scratch), totals beyond the capacities
// (a row_ptr inconsistent with the nnz the caller gave) zero the counts the
// kernels read, so nothing runs, and set totals[3].
__global__ void plan_bins_kernel(const int32_t* __restrict__ bin_count,
                                 int32_t* __restrict__ bin_cursor,
                                 const int32_t* __restrict__ slot_base,
                                 const int32_t* __restrict__ split_pos, int64_t m,
                                 int64_t* __restrict__ totals, int64_t cap_chunks,
                                 int64_t cap_split, int64_t cap_partials) {
    if (threadIdx.x == 0) {
        int64_t acc = 0;
        for (int b = kPlanBins - 1; b >= 0; --b) {
            bin_cursor[b] = static_cast<int32_t>(acc);
            acc += bin_count[b];
        }
        int64_t sacc = 0;  // split rows, longest degree bin first
        for (int b = kPlanBins - 1; b >= 0; --b) {
            bin_cursor[kPlanBins + b] = static_cast<int32_t>(sacc);
            sacc += bin_count[kPlanBins + b];
        }
        const int64_t n_split = split_pos[m], n_part = slot_base[m];
        const bool over = acc > cap_chunks || n_split > cap_split || n_part > cap_partials;
        totals[0] = over ? 0 : acc;      // chunks
        totals[1] = over ? 0 : n_split;  // split rows
        totals[2] = n_part;              // partial slots
        totals[3] = over ? 1 : 0;
    }
}

// Chunk positions are reserved per workgroup: each row takes local slots in
// an LDS histogram (its full chunks as one range, its remainder as one
// slot), then one global atomic per nonempty bin and workgroup claims the
// ranges.
__global__ __launch_bounds__(256) void plan_scatter_kernel(
    const int32_t* __restrict__ row_ptr, int64_t m, int chunk,
    const int32_t* __restrict__ slot_base, int32_t* __restrict__ bin_cursor,
    int4* __restrict__ chunks, int4* __restrict__ split, int64_t cap_chunks, int64_t cap_split) {
    __shared__ int hist[2 * kPlanBins], gbase[2 * kPlanBins];
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int b = 0, e = 0, deg = 0, full = 0, rem = 0;
    int bin_f = 0, pos_f = 0, bin_r = 0, pos_r = 0, bin_s = 0, pos_s = 0;
    if (r < m) {
        b = row_ptr[r];
        e = row_ptr[r + 1];
        deg = e - b;
        if (deg <= chunk) {
            bin_r = chunk_bin(deg);
            pos_r = atomicAdd(&hist[bin_r], 1);
            rem = -1;  // one direct chunk
        } else {
            full = deg / chunk;
            rem = deg - full * chunk;
            bin_f = chunk_bin(chunk);
            pos_f = atomicAdd(&hist[bin_f], full);
            if (rem) {
                bin_r = chunk_bin(rem);
                pos_r = atomicAdd(&hist[bin_r], 1);
            }
            bin_s = kPlanBins + chunk_bin(deg);
            pos_s = atomicAdd(&hist[bin_s], 1);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x)
        if (hist[i] > 0) gbase[i] = atomicAdd(&bin_cursor[i], hist[i]);
    __syncthreads();
    if (r >= m) return;
    const int row = static_cast<int>(r);
    // the caps only bite for a row_ptr that disagrees with the caller's nnz
    // (fixed scratch); the plan's count is then zero and nothing reads these
    if (rem < 0) {
        const int64_t at = static_cast<int64_t>(gbase[bin_r]) + pos_r;
        if (at < cap_chunks) chunks[at] = make_int4(row, b, e, -1);
        return;
    }
    const int slot0 = slot_base[r];
    for (int c = 0; c < full; ++c) {
        const int cb = b + c * chunk;
        const int64_t at = static_cast<int64_t>(gbase[bin_f]) + pos_f + c;
        if (at < cap_chunks) chunks[at] = make_int4(row, cb, cb + chunk, slot0 + c);
    }
    if (rem) {
        const int64_t at = static_cast<int64_t>(gbase[bin_r]) + pos_r;
        if (at < cap_chunks) chunks[at] = make_int4(row, b + full * chunk, e, slot0 + full);
    }
    // split rows in degree bins, longest first (agg_long_kernel's order)
    const int64_t at = static_cast<int64_t>(gbase[bin_s]) + pos_s;
    if (at < cap_split) split[at] = make_int4(row, slot0, full + (rem ? 1 : 0), deg);
}

}  // namespace

namespace {

// The plan build's temporaries, carved from the plan's scratch in the same
// layout by both phases: split_cnt[m], is_split[m], slot_base[m+1],
// split_pos[m+1], bin_count[128], bin_cursor[128], totals[4], scan temp.
struct PlanTemps {
    int32_t *split_cnt, *is_split, *slot_base, *split_pos, *bin_count, *bin_cursor;
    int64_t *totals, *scan_tmp;
};

PlanTemps carve_temps(Carver& c, int64_t m) {
    PlanTemps t;
    t.split_cnt = c.take<int32_t>(m);
    t.is_split = c.take<int32_t>(m);
    t.slot_base = c.take<int32_t>(m + 1);
    t.split_pos = c.take<int32_t>(m + 1);
    t.bin_count = c.take<int32_t>(2 * kPlanBins);  // chunk bins, then split-row bins
    t.bin_cursor = c.take<int32_t>(2 * kPlanBins);
    t.totals = c.take<int64_t>(4);
    t.scan_tmp = c.take<int64_t>(scan_temp_elems(m));
    return t;
}

PlanTemps carve_plan_temps(tg_spmm_plan_s& p, int64_t m) {
    Carver cv(nullptr, 0);
    carve_temps(cv, m);
    p.scratch.reserve(cv.bytes());
    Carver c(p.scratch.get(), p.scratch.size());
    return carve_temps(c, m);
}

}  // namespace

void build_plan_count(tg_spmm_plan_s& p, int64_t m, int64_t nnz_bound, const int32_t* row_ptr,
                      int64_t max_f, int64_t chunk, hipStream_t s, int64_t* host_totals) {
    require(m >= 0, "spmm plan: m must be >= 0");
    require(m < (int64_t(1) << 31), "spmm plan: m must be < 2^31");
    require(nnz_bound >= 0 && nnz_bound < (int64_t(1) << 31),
            "spmm plan: nnz must be < 2^31 (int32 CSR)");
    require(max_f >= 0, "spmm plan: max_f must be >= 0");
    if (chunk <= 0) chunk = kDefaultChunk;
    require(chunk <= (1 << 24), "spmm plan: chunk_nnz too large");
    TG_HIP(hipGetDevice(&p.device));
    p.m = m;
    p.nnz_bound = nnz_bound;
    p.max_f = max_f;
    p.chunk = chunk;
    p.row_ptr = row_ptr;
    p.n_chunks = p.n_split = p.n_partials = 0;
    host_totals[0] = host_totals[1] = host_totals[2] = 0;
    if (m == 0) return;
    require(row_ptr != nullptr, "spmm plan: row_ptr is null");
    const PlanTemps t = carve_plan_temps(p, m);
    fill_i32(t.bin_count, 2 * kPlanBins, 0, s);
    const unsigned nblk = static_cast<unsigned>(ceil_div(m, 256));
    plan_count_kernel<<<nblk, 256, 0, s>>>(row_ptr, m, static_cast<int>(chunk), t.split_cnt,
                                           t.is_split, t.bin_count);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(t.split_cnt, t.slot_base, m, t.scan_tmp, s);
    exclusive_scan_i32(t.is_split, t.split_pos, m, t.scan_tmp, s);
    constexpr int64_t kNoCap = INT64_MAX;  // the host sizes the buffers afterwards
    plan_bins_kernel<<<1, 64, 0, s>>>(t.bin_count, t.bin_cursor, t.slot_base, t.split_pos, m,
                                      t.totals, kNoCap, kNoCap, kNoCap);
    TG_LAUNCH_CHECK();
    TG_HIP(hipMemcpyAsync(host_totals, t.totals, 3 * sizeof(int64_t), hipMemcpyDeviceToHost, s));
}

void build_plan_finish(tg_spmm_plan_s& p, const int64_t* host_totals, hipStream_t s) {
    p.n_chunks = host_totals[0];
    p.n_split = host_totals[1];
    p.n_partials = host_totals[2];
    if (p.m == 0) return;
    const PlanTemps t = carve_plan_temps(p, p.m);
    p.chunks.reserve(static_cast<size_t>(std::max<int64_t>(p.n_chunks, 1)) * sizeof(int4));
    p.split.reserve(static_cast<size_t>(std::max<int64_t>(p.n_split, 1)) * sizeof(int4));
    // partial rows are padded to a multiple of 4 floats (128-bit access)
    if (p.n_partials > 0 && p.max_f > 0)
        p.partials.reserve(static_cast<size_t>(p.n_partials) *
                           static_cast<size_t>(round_up(p.max_f, 4)) * sizeof(float));
    const unsigned nblk = static_cast<unsigned>(ceil_div(p.m, 256));
    plan_scatter_kernel<<<nblk, 256, 0, s>>>(p.row_ptr, p.m, static_cast<int>(p.chunk),
                                             t.slot_base, t.bin_cursor,
                                             p.chunks.as<int4>(), p.split.as<int4>(),
                                             p.n_chunks, p.n_split);
    TG_LAUNCH_CHECK();
}

void build_plan(tg_spmm_plan_s& p, int64_t m, int64_t nnz_bound, const int32_t* row_ptr,
                int64_t max_f, int64_t chunk, hipStream_t s) {
    p.host_totals.reserve(4 * sizeof(int64_t));
    int64_t* tot = p.host_totals.as<int64_t>();
    build_plan_count(p, m, nnz_bound, row_ptr, max_f, chunk, s, tot);
    if (m > 0) TG_HIP(hipStreamSynchronize(s));
    build_plan_finish(p, tot, s);
}

// ---------------------------------------------------------------------------
// Several plans over consecutive row ranges of one row-pointer array (the
// per-block plans of a column-blocked copy: block b's row r at b*m + r),
// built with one launch per step for all of them and one synchronisation.
// Each step is the single-plan build's, with grid.y = the plan.
// ---------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(256) void plan_count_multi_kernel(
    const int32_t* __restrict__ row_ptr, int64_t m, int chunk, int32_t* __restrict__ split_cnt,
    int32_t* __restrict__ is_split, int32_t* __restrict__ bin_count) {
    __shared__ int32_t hist[2 * kPlanBins];
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < m) {
        const int64_t q = static_cast<int64_t>(blockIdx.y) * m + r;
        const int deg = row_ptr[q + 1] - row_ptr[q];
        const int nch = deg <= chunk ? 1 : (deg + chunk - 1) / chunk;
        split_cnt[q] = nch > 1 ? nch : 0;
        is_split[q] = nch > 1 ? 1 : 0;
        if (nch == 1) {
            atomicAdd(&hist[chunk_bin(deg)], 1);
        } else {
            const int full = deg / chunk, rem = deg - full * chunk;
            atomicAdd(&hist[chunk_bin(chunk)], full);
            if (rem) atomicAdd(&hist[chunk_bin(rem)], 1);
            atomicAdd(&hist[kPlanBins + chunk_bin(deg)], 1);
        }
    }
    __syncthreads();
    int32_t* bc = bin_count + static_cast<int64_t>(blockIdx.y) * 2 * kPlanBins;
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x)
        if (hist[i]) atomicAdd(&bc[i], hist[i]);
}

// One thread per plan: bin cursors (longest bin first) and the plan's
// totals {chunks, split rows, partial slots}, from the scans over all plans.
__global__ void plan_bins_multi_kernel(const int32_t* __restrict__ bin_count,
                                       int32_t* __restrict__ bin_cursor,
                                       const int32_t* __restrict__ slot_base,
                                       const int32_t* __restrict__ split_pos, int64_t m,
                                       int nplans, int64_t* __restrict__ totals) {
    const int b = threadIdx.x;
    if (b >= nplans) return;
    const int32_t* bc = bin_count + b * 2 * kPlanBins;
    int32_t* cur = bin_cursor + b * 2 * kPlanBins;
    int64_t acc = 0, sacc = 0;
    for (int k = kPlanBins - 1; k >= 0; --k) {
        cur[k] = static_cast<int32_t>(acc);
        acc += bc[k];
        cur[kPlanBins + k] = static_cast<int32_t>(sacc);  // split rows, longest first
        sacc += bc[kPlanBins + k];
    }
    const int64_t lo = static_cast<int64_t>(b) * m, hi = lo + m;
    totals[4 * b + 0] = acc;
    totals[4 * b + 1] = split_pos[hi] - split_pos[lo];
    totals[4 * b + 2] = slot_base[hi] - slot_base[lo];
    totals[4 * b + 3] = 0;
}

struct MultiPlanOut {
    int4* chunks[kMaxMultiPlans];
    int4* split[kMaxMultiPlans];
};

__global__ __launch_bounds__(256) void plan_scatter_multi_kernel(
    const int32_t* __restrict__ row_ptr, int64_t m, int chunk,
    const int32_t* __restrict__ slot_base, int32_t* __restrict__ bin_cursor, MultiPlanOut out) {
    __shared__ int hist[2 * kPlanBins], gbase[2 * kPlanBins];
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t lo = static_cast<int64_t>(blockIdx.y) * m;
    int b = 0, e = 0, deg = 0, full = 0, rem = 0;
    int bin_f = 0, pos_f = 0, bin_r = 0, pos_r = 0, bin_s = 0, pos_s = 0;
    if (r < m) {
        b = row_ptr[lo + r];
        e = row_ptr[lo + r + 1];
        deg = e - b;
        if (deg <= chunk) {
            bin_r = chunk_bin(deg);
            pos_r = atomicAdd(&hist[bin_r], 1);
            rem = -1;  // one direct chunk
        } else {
            full = deg / chunk;
            rem = deg - full * chunk;
            bin_f = chunk_bin(chunk);
            pos_f = atomicAdd(&hist[bin_f], full);
            if (rem) {
                bin_r = chunk_bin(rem);
                pos_r = atomicAdd(&hist[bin_r], 1);
            }
            bin_s = kPlanBins + chunk_bin(deg);
            pos_s = atomicAdd(&hist[bin_s], 1);
        }
    }
    __syncthreads();
    int32_t* cur = bin_cursor + static_cast<int64_t>(blockIdx.y) * 2 * kPlanBins;
    for (int i = threadIdx.x; i < 2 * kPlanBins; i += blockDim.x)
        if (hist[i] > 0) gbase[i] = atomicAdd(&cur[i], hist[i]);
    __syncthreads();
    if (r >= m) return;
    int4* chunks = out.chunks[blockIdx.y];
    const int row = static_cast<int>(r);
    if (rem < 0) {
        chunks[gbase[bin_r] + pos_r] = make_int4(row, b, e, -1);
        return;
    }
    // slots and split positions count from the plan's first row
    const int slot0 = slot_base[lo + r] - slot_base[lo];
    for (int c = 0; c < full; ++c) {
        const int cb = b + c * chunk;
        chunks[gbase[bin_f] + pos_f + c] = make_int4(row, cb, cb + chunk, slot0 + c);
    }
    if (rem) chunks[gbase[bin_r] + pos_r] = make_int4(row, b + full * chunk, e, slot0 + full);
    // split rows in degree bins, longest first (agg_long_kernel's order)
    out.split[blockIdx.y][gbase[bin_s] + pos_s] = make_int4(row, slot0, full + (rem ? 1 : 0), deg);
}

struct MultiTemps {
    int32_t *split_cnt, *is_split, *slot_base, *split_pos, *bin_count, *bin_cursor;
    int64_t *totals, *scan_tmp;
};

MultiTemps carve_multi(Carver& c, int64_t rows, int nplans) {
    MultiTemps t;
    t.split_cnt = c.take<int32_t>(rows);
    t.is_split = c.take<int32_t>(rows);
    t.slot_base = c.take<int32_t>(rows + 1);
    t.split_pos = c.take<int32_t>(rows + 1);
    t.bin_count = c.take<int32_t>(static_cast<int64_t>(nplans) * 2 * kPlanBins);
    t.bin_cursor = c.take<int32_t>(static_cast<int64_t>(nplans) * 2 * kPlanBins);
    t.totals = c.take<int64_t>(4 * static_cast<int64_t>(nplans));
    t.scan_tmp = c.take<int64_t>(scan_temp_elems(rows));
    return t;
}

}  // namespace

void build_plans_multi(tg_spmm_plan_s* const* plans, int nplans, int64_t m,
                       int64_t nnz_bound, const int32_t* row_ptr, int64_t max_f, int64_t chunk,
                       DeviceBuffer& scratch, int64_t* host_totals, hipStream_t s) {
    require(nplans >= 1 && nplans <= kMaxMultiPlans, "spmm plans: 1 to 64 plans per build");
    require(m >= 1 && static_cast<int64_t>(nplans) * m < (int64_t(1) << 31),
            "spmm plans: plans x rows must be < 2^31");
    require(nnz_bound >= 0 && nnz_bound < (int64_t(1) << 31),
            "spmm plans: nnz must be < 2^31 (int32 CSR)");
    require(row_ptr != nullptr && max_f >= 0, "spmm plans: bad arguments");
    if (chunk <= 0) chunk = kDefaultChunk;
    require(chunk <= (1 << 24), "spmm plans: chunk_nnz too large");
    const int64_t rows = static_cast<int64_t>(nplans) * m;
    Carver cv(nullptr, 0);
    carve_multi(cv, rows, nplans);
    scratch.reserve(cv.bytes());
    Carver c(scratch.get(), scratch.size());
    const MultiTemps t = carve_multi(c, rows, nplans);
    fill_i32(t.bin_count, static_cast<int64_t>(nplans) * 2 * kPlanBins, 0, s);
    const dim3 grid(static_cast<unsigned>(ceil_div(m, 256)), static_cast<unsigned>(nplans));
    plan_count_multi_kernel<<<grid, 256, 0, s>>>(row_ptr, m, static_cast<int>(chunk),
                                                 t.split_cnt, t.is_split, t.bin_count);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(t.split_cnt, t.slot_base, rows, t.scan_tmp, s);
    exclusive_scan_i32(t.is_split, t.split_pos, rows, t.scan_tmp, s);
    plan_bins_multi_kernel<<<1, kMaxMultiPlans, 0, s>>>(t.bin_count, t.bin_cursor, t.slot_base,
                                                        t.split_pos, m, nplans, t.totals);
    TG_LAUNCH_CHECK();
    TG_HIP(hipMemcpyAsync(host_totals, t.totals, 4 * nplans * sizeof(int64_t),
                          hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    int device = 0;
    TG_HIP(hipGetDevice(&device));
    MultiPlanOut out{};
    for (int b = 0; b < nplans; ++b) {
        tg_spmm_plan_s& p = *plans[b];
        p.device = device;
        p.m = m;
        p.nnz_bound = nnz_bound;
        p.max_f = max_f;
        p.chunk = chunk;
        p.row_ptr = row_ptr + static_cast<int64_t>(b) * m;
        p.n_chunks = host_totals[4 * b + 0];
        p.n_split = host_totals[4 * b + 1];
        p.n_partials = host_totals[4 * b + 2];
        p.chunks.reserve(static_cast<size_t>(std::max<int64_t>(p.n_chunks, 1)) * sizeof(int4));
        p.split.reserve(static_cast<size_t>(std::max<int64_t>(p.n_split, 1)) * sizeof(int4));
        if (p.n_partials > 0 && p.max_f > 0)
            p.partials.reserve(static_cast<size_t>(p.n_partials) *
                               static_cast<size_t>(round_up(p.max_f, 4)) * sizeof(float));
        out.chunks[b] = p.chunks.as<int4>();
        out.split[b] = p.split.as<int4>();
    }
    plan_scatter_multi_kernel<<<grid, 256, 0, s>>>(row_ptr, m, static_cast<int>(chunk),
                                                   t.slot_base, t.bin_cursor, out);
    TG_LAUNCH_CHECK();
}

LaneLayout choose_layout(int64_t f, int vec) {
    LaneLayout L{};
    L.vec = vec;
    const int64_t nvec = ceil_div(std::max<int64_t>(f, 1), vec);
    // One vector per lane; rows wider than a wavefront's 64 vectors are cut
    // into 64-lane column tiles (grid.y), each re-reading the chunk's
    // indices.  Measured at config D, F=512: two tiles with 16 gathers in
    // flight per lane take 15.5 ms, one tile of two vectors per lane (8 in
    // flight) 16.7 ms.
    int lpr = 4;
    while (lpr < nvec && lpr < 64) lpr <<= 1;
    L.lpr = lpr;
    L.vpl = 1;
    L.tile = L.lpr * L.vpl * L.vec;
    L.n_tiles = static_cast<int>(ceil_div(std::max<int64_t>(f, 1), L.tile));
    return L;
}

int pick_vec(int64_t f, std::initializer_list<int64_t> lds,
             std::initializer_list<const void*> ptrs) {
    for (int v : {4, 2}) {
        bool ok = (f % v) == 0;
        for (int64_t ld : lds) ok = ok && (ld % v) == 0;
        for (const void* p : ptrs)
            ok = ok && (reinterpret_cast<uintptr_t>(p) % (sizeof(float) * v)) == 0;
        if (ok) return v;
    }
    return 1;
}

int pick_load_vec(int64_t f, int64_t ldb, const void* b) {
    for (int v : {4, 2}) {
        if (ldb % v == 0 && round_up(f, v) <= ldb &&
            reinterpret_cast<uintptr_t>(b) % (sizeof(float) * v) == 0)
            return v;
    }
    return 1;
}

// ---------------------------------------------------------------------------
// Aggregation kernels
// ---------------------------------------------------------------------------
namespace {

template <int VEC>
struct VecOf;
template <>
struct VecOf<1> { using T = float; };
template <>
struct VecOf<2> { using T = float2; };
template <>
struct VecOf<4> { using T = float4; };

template <int VEC>
__device__ __forceinline__ void load_vec(const float* p, float (&x)[VEC]) {
    using T = typename VecOf<VEC>::T;
    T t = *reinterpret_cast<const T*>(p);
    const float* q = reinterpret_cast<const float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = q[k];
}

// Non-temporal forms for the aggregation's output rows, which a pass reads
// (a column-block pass continuing a chain) and writes once: streamed, they
// do not evict the gathered lines from L2 (config-E forwards 1-2% faster).
template <int VEC>
struct NVec;
template <>
struct NVec<1> { typedef float T; };
template <>
struct NVec<2> { typedef float T __attribute__((ext_vector_type(2))); };
template <>
struct NVec<4> { typedef float T __attribute__((ext_vector_type(4))); };

template <int VEC>
__device__ __forceinline__ void store_vec_nt(float* p, const float (&x)[VEC]) {
    typename NVec<VEC>::T t;
    float* q = reinterpret_cast<float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) q[k] = x[k];
    __builtin_nontemporal_store(t, reinterpret_cast<typename NVec<VEC>::T*>(p));
}

template <int VEC>
__device__ __forceinline__ void load_vec_nt(const float* p, float (&x)[VEC]) {
    const typename NVec<VEC>::T t =
        __builtin_nontemporal_load(reinterpret_cast<const typename NVec<VEC>::T*>(p));
    const float* q = reinterpret_cast<const float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = q[k];
}

template <int VEC>
__device__ __forceinline__ void store_vec(float* p, const float (&x)[VEC]) {
    using T = typename VecOf<VEC>::T;
    T t;
    float* q = reinterpret_cast<float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) q[k] = x[k];
    *reinterpret_cast<T*>(p) = t;
}

__device__ __forceinline__ float apply_act(float x, int act, int post, int exact_exp = 0) {
    if (act == TG_ACT_RELU) x = (0.0f < x) ? x : 0.0f;
    if (post == TG_POST_RELU) {
        x = (0.0f < x) ? x : 0.0f;
    } else if (post == TG_POST_ELU) {
        if (x < 0.0f) x = 1.0f * ((exact_exp ? exp_rn(x) : expf(x)) - 1.0f);
    }
    return x;
}

// The self term's vector at column fo of row `row` (row-major or
// tile-major; a vector never crosses a 32-column tile).
__device__ __forceinline__ const float* self_row(const AggEpilogue& epi, int row, int64_t fo) {
    return epi.self_tile_stride > 0
               ? epi.self + (fo >> 5) * epi.self_tile_stride + static_cast<int64_t>(row) * 32 +
                     (fo & 31)
               : epi.self + static_cast<int64_t>(row) * epi.ld_self + fo;
}

// add_prev: x is the sum of this pass only, to be added to the row's value
// stored by the earlier column-block passes (split rows); an unsplit row's
// pass starts its chain from that value instead (see agg_chunk_kernel).
template <int VEC>
__device__ __forceinline__ void finish_store(float (&x)[VEC], int row, int deg, int64_t fo,
                                             int64_t f, float* __restrict__ c, int64_t ldc,
                                             const AggEpilogue& epi, bool add_prev) {
    if (add_prev) {
        // the sum of the earlier column-block passes, then this pass's
        const float* prev = c + static_cast<int64_t>(row) * ldc + fo;
        if (epi.vec_io) {
            float t[VEC];
            load_vec<VEC>(prev, t);
#pragma unroll
            for (int k = 0; k < VEC; ++k) x[k] = t[k] + x[k];
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                if (fo + k < f) x[k] = prev[k] + x[k];
        }
    }
    if (epi.deg_rp) deg = epi.deg_rp[row + 1] - epi.deg_rp[row];
    if (epi.mean && deg > 0) {
        const float inv = 1.0f / static_cast<float>(deg);
#pragma unroll
        for (int k = 0; k < VEC; ++k) x[k] *= inv;
    }
    if (epi.row_scale) {
        const float* sc = epi.row_scale + static_cast<int64_t>(row) * epi.scale_ld;
#pragma unroll
        for (int k = 0; k < VEC; ++k) x[k] *= sc[(fo + k < f ? fo + k : fo) / epi.scale_cols];
    }
    if (!epi.vec_io) {
        // element by element, within the f valid columns (the output or the
        // epilogue operands are not aligned to the access width)
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if (fo + k >= f) break;
            float v = x[k];
            if (epi.self) v += self_row(epi, row, fo)[k];
            if (epi.bias) v += epi.bias[fo + k];
            c[static_cast<int64_t>(row) * ldc + fo + k] = apply_act(v, epi.act, epi.post, epi.exact_exp);
        }
        return;
    }
    if (epi.self) {
        float t[VEC];
        load_vec<VEC>(self_row(epi, row, fo), t);
#pragma unroll
        for (int k = 0; k < VEC; ++k) x[k] += t[k];
    }
    if (epi.bias) {
        float t[VEC];
        load_vec<VEC>(epi.bias + fo, t);
#pragma unroll
        for (int k = 0; k < VEC; ++k) x[k] += t[k];
    }
    if (epi.act | epi.post) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) x[k] = apply_act(x[k], epi.act, epi.post, epi.exact_exp);
    }
    store_vec_nt<VEC>(c + static_cast<int64_t>(row) * ldc + fo, x);
}

// kAggAttn: GAT's attention weights, computed per entry inside the pass
// (AggEpilogue.att_*), then accumulated as kAggWeighted's.
// kAggSumTail: kAggSum whose chunks' last, partial batches gather nothing
// for the slots past the chunk's end (AggEpilogue.mask_tail).
enum { kAggWeighted = 0, kAggSum = 1, kAggMax = 2, kAggAttn = 3, kAggSumTail = 4 };

// One step of a row's reduction: fma with the edge weight (SpMM's value,
// ops.cpp:266-287, or a GAT attention weight), a plain add (SAGE mean,
// layers.cpp:604-620), or the element-wise max written as
// std::max(acc, x) = (acc < x) ? x : acc (layers.cpp:398-417).
template <int MODE>
__device__ __forceinline__ float combine(float acc, float x, float w) {
    if constexpr (MODE == kAggWeighted || MODE == kAggAttn) return __builtin_fmaf(w, x, acc);
    if constexpr (MODE == kAggSum || MODE == kAggSumTail) return acc + x;
    return (acc < x) ? x : acc;
}

// Gathers in flight per lane (row vectors of B loaded before they are used):
// 16 single vectors (measured 2-4% faster than 8 on the column-blocked
// passes and the narrow SpMM, at lower occupancy); VPL > 1 layouts (no longer
// chosen) would keep 8 pairs or 4 quads.
template <int VPL>
struct Unroll {
    static constexpr int value = VPL == 1 ? 16 : VPL == 2 ? 8 : 4;
};


template <int VEC, int LPR, int VPL, int MODE>
__global__ __launch_bounds__(256, 4) void agg_chunk_kernel(
    const int4* __restrict__ chunks, int64_t n_chunks, const int64_t* __restrict__ n_chunks_dev,
    const int32_t* __restrict__ ci,
    const float* __restrict__ av, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, float* __restrict__ partials, int64_t ldp, int64_t f,
    AggEpilogue epi) {
    constexpr int GPB = 256 / LPR;
    constexpr int U = Unroll<VPL>::value;
    constexpr int TILE = LPR * VPL * VEC;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    // a plan in fixed scratch: the grid covers an upper bound, the count is
    // in device memory
    if (cid >= (n_chunks_dev ? *n_chunks_dev : n_chunks)) return;
    const int4 ch = chunks[cid];
    if (epi.skip_empty && ch.z == ch.y) return;  // the row keeps its value in C
    if (epi.long_rows && ch.w >= 0) return;      // a split row: agg_long_kernel's
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    // attention weights: the row's score, max and 1/sum for the tile's head
    // (every tile lies in one head's columns); dst scores of that head
    float att_s = 0.0f, att_m = 0.0f, att_r = 0.0f;
    const float* att_d = nullptr;
    if constexpr (MODE == kAggAttn) {
        const int64_t h = fbase / epi.w_head_cols;
        const int64_t o = static_cast<int64_t>(ch.x) * epi.att_heads + h;
        att_s = epi.att_src[o];
        att_m = epi.att_max[o];
        att_r = epi.att_rinv[o];
        att_d = epi.att_dst + h;
    }

    int64_t fo[VPL], fl[VPL];
    bool ok[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        fo[v] = fbase + static_cast<int64_t>(l + v * LPR) * VEC;
        ok[v] = fo[v] < f;
        // lanes past f load the tile's first vector (the same cache line as
        // the tile's valid columns; fbase < f), never stored
        fl[v] = ok[v] ? fo[v] : fbase;
    }
    float acc[VPL][VEC];
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[v][k] = MODE == kAggMax ? -INFINITY : 0.0f;
    // A column-block pass after the first continues an unsplit row's chain
    // from the value the earlier passes stored.  With the row's entries in
    // block order equal to their nonzero order (the host checks), the passes
    // together run the row's one chain in nonzero order, as unblocked.
    const bool chain = epi.acc && ch.w < 0;
    if (chain) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            if (!ok[v]) continue;
            const float* prev = C + static_cast<int64_t>(ch.x) * ldc + fo[v];
            if (epi.vec_io) {
                load_vec_nt<VEC>(prev, acc[v]);
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[v][k] = fo[v] + k < f ? prev[k] : 0.0f;
            }
        }
    }

    // The chunk's entries are walked in batches of BE = max(LPR, U): each
    // lane of the group loads CPL consecutive (col, val) pairs of the batch
    // with one coalesced access, and the group broadcasts them with
    // shuffles, so the per-edge cost is the row gather alone.  Edges stay in
    // nonzero order (entry t of a batch is lane t / CPL, slot t % CPL).
    // The next batch's pairs are loaded once the current batch's first
    // gathers are issued, so their latency overlaps the gathers'.
    constexpr int CPL = U > LPR ? U / LPR : 1;
    constexpr int BE = LPR * CPL;
    const int e = ch.z;
    // Gather address = the lane's base (B + its column offset) + col * row
    // pitch in bytes: one 32 x 32 -> 64-bit multiply-add per gather (col >= 0;
    // the host keeps the pitch in bytes below 2^32).  A tile-major B puts
    // column c in tile c / 32 at offset c % 32 (a 64-column group spans two
    // tiles).
    const char* bl[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v)
        bl[v] = reinterpret_cast<const char*>(
            epi.b_tile_stride > 0 ? B + (fl[v] >> 5) * epi.b_tile_stride + (fl[v] & 31)
                                  : B + fl[v]);
    const uint32_t pitch = static_cast<uint32_t>(ldb) * 4u;
    int ncl[CPL];
    float nwl[CPL];
    auto fetch = [&](int base) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int idx = base + l * CPL + j;
            ncl[j] = idx < e ? (epi.ci16 ? static_cast<int>(epi.ci16[idx]) : ci[idx]) : 0;
            nwl[j] = 1.0f;
            if constexpr (MODE == kAggWeighted) nwl[j] = idx < e ? av[idx] : 0.0f;
        }
    };
    fetch(ch.y);
    const int att_stride = epi.att_heads;
    for (int base = ch.y; base < e; base += BE) {
        int cl[CPL];
        float wl[CPL], dl[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            cl[j] = ncl[j];
            wl[j] = nwl[j];
            // the batch's destination scores, loaded before its row gathers
            // so that their latency overlaps the gathers'
            if constexpr (MODE == kAggAttn)
                dl[j] = att_d[static_cast<int64_t>(cl[j]) * att_stride];
        }
        // U gathers in flight per step; in the chunk's last, partial batch
        // the slots past its end are not accumulated (and gather row 0, in
        // bounds since cl is 0 there, or nothing; see below).
        if constexpr (LPR == 16 || LPR == 4) {
            const int cnt = e - base < BE ? e - base : BE;
            // slot s0 + u of the batch is entry (s0 + u) % CPL of lane (s0 + u) / CPL:
            // compile-time lanes, broadcast without LDS (group_bcast)
            static_for<0, BE / U>([&](auto sc) {
                constexpr int s0 = decltype(sc)::value * U;
                if (s0 < cnt) {  // uniform across the group: no early exit in the unrolled body
                    int col[U];
                    float w[U];
                    static_for<0, U>([&](auto uc) {
                        constexpr int u = decltype(uc)::value;
                        col[u] = group_bcast<LPR, (s0 + u) / CPL>(cl[(s0 + u) % CPL]);
                        w[u] = 1.0f;
                        if constexpr (MODE == kAggWeighted)
                            w[u] = group_bcast<LPR, (s0 + u) / CPL>(wl[(s0 + u) % CPL]);
                    });
                    // kAggSumTail (the fast column-blocked GCN and SAGE passes):
                    // slots past the chunk's end gather nothing, their lanes
                    // masked off (config-E GCN / SAGE forwards 1% faster); the
                    // other modes gather row 0 there (the per-slot branches cost
                    // more than they save on config D's short rows, in the GAT
                    // passes and on exact SAGE's long chunks, 4%)
                    float bv[U][VPL][VEC];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(col[u])) * pitch;
                        if (MODE != kAggSumTail || s0 + u < cnt) {
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
                                load_vec<VEC>(reinterpret_cast<const float*>(bl[v] + off), bv[u][v]);
                        } else {
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k) bv[u][v][k] = 0.0f;
                        }
                    }
                    if (s0 == 0) fetch(base + BE);
                    if constexpr (MODE == kAggAttn) {
                        // alpha_ij = exp(LeakyReLU(s_i + d_j) - max_i) * (1/sum_i)
                        // (layers.cpp:1068-1090), once per entry and head
                        if (s0 == 0) {
#pragma unroll
                            for (int j = 0; j < CPL; ++j) {
                                const float x = att_s + dl[j];
                                const float t = ((x >= 0.0f) ? x : epi.att_slope * x) - att_m;
                                wl[j] = (epi.exact_exp ? exp_rn(t) : expf(t)) * att_r;
                            }
                        }
                    }
                    // the weight of slot u: attention weights are broadcast at
                    // their fma (not all U held at once: fewer live registers)
                    auto wt = [&](auto uc) {
                        constexpr int u = decltype(uc)::value;
                        if constexpr (MODE == kAggAttn)
                            return group_bcast<LPR, (s0 + u) / CPL>(wl[(s0 + u) % CPL]);
                        else
                            return w[u];
                    };
                    if (cnt == BE) {  // a full batch: every slot is an entry
                        static_for<0, U>([&](auto uc) {
                            constexpr int u = decltype(uc)::value;
                            const float wu = wt(uc);
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k)
                                    acc[v][k] = combine<MODE>(acc[v][k], bv[u][v][k], wu);
                        });
                    } else {
                        static_for<0, U>([&](auto uc) {
                            constexpr int u = decltype(uc)::value;
                            const bool valid = s0 + u < cnt;  // a select, not a branch
                            const float wu = wt(uc);
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k) {
                                    const float nx = combine<MODE>(acc[v][k], bv[u][v][k], wu);
                                    acc[v][k] = valid ? nx : acc[v][k];
                                }
                        });
                    }
                }
            });
        } else {
            // other group widths: runtime-lane shuffles (the compile-time form
            // measured 2-3% slower for the F=128 / F=512 SpMM, no faster at 8)
            const int cnt = e - base < BE ? e - base : BE;
#pragma unroll
            for (int s0 = 0; s0 < BE; s0 += U) {
                if (s0 < cnt) {  // uniform across the group: no early exit in the unrolled body
                    int col[U];
                    float w[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        col[u] = __shfl(cl[(s0 + u) % CPL], (s0 + u) / CPL, LPR);
                        w[u] = 1.0f;
                        if constexpr (MODE == kAggWeighted)
                            w[u] = __shfl(wl[(s0 + u) % CPL], (s0 + u) / CPL, LPR);
                    }
                    // kAggSumTail (the fast column-blocked GCN and SAGE passes):
                    // slots past the chunk's end gather nothing, their lanes
                    // masked off (config-E GCN / SAGE forwards 1% faster); the
                    // other modes gather row 0 there (the per-slot branches cost
                    // more than they save on config D's short rows, in the GAT
                    // passes and on exact SAGE's long chunks, 4%)
                    float bv[U][VPL][VEC];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(col[u])) * pitch;
                        if (MODE != kAggSumTail || s0 + u < cnt) {
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
                                load_vec<VEC>(reinterpret_cast<const float*>(bl[v] + off), bv[u][v]);
                        } else {
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k) bv[u][v][k] = 0.0f;
                        }
                    }
                    if (s0 == 0) fetch(base + BE);
                    if constexpr (MODE == kAggAttn) {
                        // alpha_ij = exp(LeakyReLU(s_i + d_j) - max_i) * (1/sum_i)
                        // (layers.cpp:1068-1090), once per entry and head
                        if (s0 == 0) {
#pragma unroll
                            for (int j = 0; j < CPL; ++j) {
                                const float x = att_s + dl[j];
                                const float t = ((x >= 0.0f) ? x : epi.att_slope * x) - att_m;
                                wl[j] = (epi.exact_exp ? exp_rn(t) : expf(t)) * att_r;
                            }
                        }
                    }
                    // the weight of slot u: attention weights are broadcast at
                    // their fma (not all U held at once: fewer live registers)
                    auto wt = [&](int u) {
                        if constexpr (MODE == kAggAttn)
                            return __shfl(wl[(s0 + u) % CPL], (s0 + u) / CPL, LPR);
                        else
                            return w[u];
                    };
                    if (cnt == BE) {  // a full batch: every slot is an entry
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const float wu = wt(u);
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k)
                                    acc[v][k] = combine<MODE>(acc[v][k], bv[u][v][k], wu);
                        }
                    } else {
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const bool valid = s0 + u < cnt;  // a select, not a branch
                            const float wu = wt(u);
#pragma unroll
                            for (int v = 0; v < VPL; ++v)
#pragma unroll
                                for (int k = 0; k < VEC; ++k) {
                                    const float nx = combine<MODE>(acc[v][k], bv[u][v][k], wu);
                                    acc[v][k] = valid ? nx : acc[v][k];
                                }
                        }
                    }
                }
            }
        }
    }

    if (ch.w < 0) {
        if (MODE == kAggMax && ch.z == ch.y) {
            // an empty row aggregates to 0 (layers.cpp:377-380)
#pragma unroll
            for (int v = 0; v < VPL; ++v)
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[v][k] = 0.0f;
        }
#pragma unroll
        for (int v = 0; v < VPL; ++v)
            if (ok[v]) finish_store<VEC>(acc[v], ch.x, ch.z - ch.y, fo[v], f, C, ldc, epi, false);
    } else {
        float* prow = partials + static_cast<int64_t>(ch.w) * ldp;
#pragma unroll
        for (int v = 0; v < VPL; ++v)
            if (ok[v]) store_vec<VEC>(prow + fo[v], acc[v]);
    }
}

// The fast column-blocked passes' kernel (kAggSumTail over 16-bit block
// indices, 8-lane groups of 32 columns): agg_chunk_kernel<4, 8, 1,
// kAggSumTail>'s arithmetic, with the index stream read through scalar loads.
//
// Vector loads of a compute unit return in issue order, so an index load
// that misses to the MALL or HBM holds back the L2-resident gathers issued
// after it, by any wavefront of that unit.  Scalar loads return through the
// scalar cache instead: a gather probe at a 4 MB block (32,768 rows of
// 128 B) with a 537 MB index stream moved 25.8 TB/s with scalar index loads
// against 22.0 with vector ones (a producer wavefront streaming the indices
// into LDS through vector loads: 22.9).
//
// The wavefront walks its eight chunks in a uniform loop of 16-entry batches
// over dword-aligned positions (a chunk starting at an odd entry masks its
// first slot).  Each batch, one scalar load per group brings 8 dwords (16
// indices) and v_writelane spreads them as the vector path holds them (lane
// p of a group: entries 2p, 2p + 1), for the same shuffles; the next batch's
// scalar loads are issued after the current gathers.  A finished group
// reloads its last batch (unused), so every load stays within the chunk's
// batches, at most 15 entries past its end (the blocked copy keeps 64 bytes
// of padding after its indices).
__device__ __forceinline__ uint32_t put_group(const uint32_t (&d)[8], int gg, uint32_t v) {
    switch (gg) {  // gg is a compile-time constant after unrolling
#define TG_PUT(G)                                                                      \
    case G:                                                                            \
        v = write_lane<8 * G + 0>(d[0], v);                                            \
        v = write_lane<8 * G + 1>(d[1], v);                                            \
        v = write_lane<8 * G + 2>(d[2], v);                                            \
        v = write_lane<8 * G + 3>(d[3], v);                                            \
        v = write_lane<8 * G + 4>(d[4], v);                                            \
        v = write_lane<8 * G + 5>(d[5], v);                                            \
        v = write_lane<8 * G + 6>(d[6], v);                                            \
        v = write_lane<8 * G + 7>(d[7], v);                                            \
        break;
        TG_PUT(0) TG_PUT(1) TG_PUT(2) TG_PUT(3) TG_PUT(4) TG_PUT(5) TG_PUT(6) TG_PUT(7)
#undef TG_PUT
    }
    return v;
}

// A raw buffer load of 16 bytes at byte offset `off` of the range the
// descriptor covers; an offset past the range's end reads zeros without a
// memory access.  Descriptor: base address, stride 0, num_records = the
// range's bytes, and the gfx9 data-format word.
typedef int BufRsrc __attribute__((ext_vector_type(4)));
typedef float Float4v __attribute__((ext_vector_type(4)));
__device__ Float4v raw_buffer_load_f32x4(BufRsrc rsrc, uint32_t voffset, uint32_t soffset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.load.v4f32");

__device__ __forceinline__ BufRsrc buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    BufRsrc r;
    r.x = static_cast<int>(a & 0xFFFFFFFFu);
    r.y = static_cast<int>(a >> 32);  // stride 0
    r.z = static_cast<int>(bytes);
    r.w = 0x00020000;
    return r;
}

// BUF = 0: gathers through 64-bit addresses, slots outside the chunk
// skipped and masked; BUF = 1 (tile-major B) / 2 (row-major B with rows of
// less than 2^16 bytes): gathers through buffer loads over B's first
// min(b_rows, 65535) rows, where the slots outside the chunk take column
// 0xFFFF, past that range, and read zeros -- added unconditionally (the
// sums start from +0 or an earlier pass's sum, never -0, so adding +0
// changes no bit).  Fewer instructions per gathered row (the passes issue
// their gathers at a higher rate).
template <int BUF>
__global__ __launch_bounds__(256, 4) void agg_sidx_kernel(
    const int4* __restrict__ chunks, int64_t n_chunks, const int64_t* __restrict__ n_chunks_dev,
    const float* __restrict__ B, int64_t ldb, float* __restrict__ C, int64_t ldc,
    float* __restrict__ partials, int64_t ldp, int64_t f, AggEpilogue epi) {
    static_assert(BUF >= 0 && BUF <= 2, "gather mode");
    constexpr int LPR = 8, VEC = 4, U = 16;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + g;
    const int64_t nch = n_chunks_dev ? *n_chunks_dev : n_chunks;
    // groups past the plan's end, and empty chunks of a middle pass, take
    // part in the wavefront's loop with no entries and store nothing
    int4 ch = make_int4(0, 0, 0, -1);
    bool active = cid < nch;
    if (active) ch = chunks[cid];
    if (active && epi.skip_empty && ch.z == ch.y) active = false;
    if (active && epi.long_rows && ch.w >= 0) active = false;  // agg_long_kernel's row
    if (!active) ch = make_int4(0, 0, 0, -1);
    if (__builtin_amdgcn_readfirstlane(__ballot(active) == 0 ? 1 : 0)) return;

    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * (LPR * VEC);
    const int64_t fo = fbase + static_cast<int64_t>(l) * VEC;
    const bool ok = fo < f;
    const int64_t fl = ok ? fo : fbase;
    float acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
    if (active && epi.acc && ch.w < 0 && ok) {
        // continue the row's chain from the earlier passes' value
        const float* prev = C + static_cast<int64_t>(ch.x) * ldc + fo;
        if (epi.vec_io) {
            load_vec_nt<VEC>(prev, acc);
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k) acc[k] = fo + k < f ? prev[k] : 0.0f;
        }
    }
    const char* bl = reinterpret_cast<const char*>(
        epi.b_tile_stride > 0 ? B + (fl >> 5) * epi.b_tile_stride + (fl & 31) : B + fl);
    const uint32_t pitch = static_cast<uint32_t>(ldb) * 4u;
    // the buffer modes: the tile's first column of B's first row (the same
    // for the whole workgroup) and the lane's columns as an offset in a row
    BufRsrc rsrc{};
    uint32_t laneoff = 0;
    if constexpr (BUF != 0) {
        const int64_t rows = epi.b_rows < 65535 ? epi.b_rows : 65535;
        const float* bt = BUF == 1 ? B + static_cast<int64_t>(blockIdx.y) * epi.b_tile_stride
                                   : B + fbase;
        rsrc = buffer_rsrc(bt, static_cast<uint32_t>(rows * pitch));
        laneoff = ok ? static_cast<uint32_t>(l) * 16u : 0u;
    }

    // the group's batches: 16 entries each from the dword-aligned start
    const int a = ch.y & ~1;
    const int nb = ch.z > ch.y ? (ch.z - a + 15) >> 4 : 0;
    int nmax = 0;
#pragma unroll
    for (int gg = 0; gg < kWave / LPR; ++gg) {
        const int x = __builtin_amdgcn_readlane(nb, gg * LPR);
        nmax = x > nmax ? x : nmax;
    }
    const uint32_t* cw = reinterpret_cast<const uint32_t*>(epi.ci16);
    // dword offset of batch t of the lane's group (its last batch once done;
    // 0 for a group with none)
    auto batch_off = [&](int t) { return nb > 0 ? (a >> 1) + 8 * (t < nb ? t : nb - 1) : 0; };
    auto load_batch = [&](int t, uint32_t (&d)[kWave / LPR][8]) {
        const int o = batch_off(t);
#pragma unroll
        for (int gg = 0; gg < kWave / LPR; ++gg) {
            const int og = __builtin_amdgcn_readlane(o, gg * LPR);
#pragma unroll
            for (int p = 0; p < 8; ++p) d[gg][p] = cw[og + p];
        }
    };
    uint32_t d[kWave / LPR][8];
    uint32_t packed = 0;
    load_batch(0, d);
#pragma unroll
    for (int gg = 0; gg < kWave / LPR; ++gg) packed = put_group(d[gg], gg, packed);

    for (int t = 0; t < nmax; ++t) {
        // slots [lo, cnt) of this batch are the group's entries
        const int base = a + 16 * t;
        const int lo = ch.y - base, cnt = ch.z - base;
        float bv[U][VEC];
        if constexpr (BUF == 0) {
            const int c0 = static_cast<int>(packed & 0xFFFFu);
            const int c1 = static_cast<int>(packed >> 16);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int col = __shfl((u & 1) ? c1 : c0, u >> 1, LPR);
                if (u >= lo && u < cnt) {
                    const uint64_t off =
                        static_cast<uint64_t>(static_cast<uint32_t>(col)) * pitch;
                    load_vec<VEC>(reinterpret_cast<const float*>(bl + off), bv[u]);
                } else {
#pragma unroll
                    for (int k = 0; k < VEC; ++k) bv[u][k] = 0.0f;
                }
            }
        } else {
            // the lane's two slots 2l and 2l + 1: outside the chunk, column
            // 0xFFFF (past the range: zeros)
            const uint32_t keep = (2 * l >= lo && 2 * l < cnt ? 0x0000FFFFu : 0u) |
                                  (2 * l + 1 >= lo && 2 * l + 1 < cnt ? 0xFFFF0000u : 0u);
            const uint32_t pk = (packed & keep) | ~keep;
            const uint32_t c0 = pk & 0xFFFFu, c1 = pk >> 16;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t col = static_cast<uint32_t>(__shfl((u & 1) ? c1 : c0, u >> 1, LPR));
                const uint32_t off = BUF == 1 ? (col << 7) + laneoff : __umul24(col, pitch) + laneoff;
                const Float4v v = raw_buffer_load_f32x4(rsrc, off, 0u, 0);
                bv[u][0] = v.x;
                bv[u][1] = v.y;
                bv[u][2] = v.z;
                bv[u][3] = v.w;
            }
        }
        // the next batch's indices, behind this batch's gathers
        __builtin_amdgcn_sched_barrier(0);
        load_batch(t + 1, d);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (BUF == 0) {
                const bool valid = u >= lo && u < cnt;  // a select, not a branch
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const float nx = acc[k] + bv[u][k];
                    acc[k] = valid ? nx : acc[k];
                }
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[k] += bv[u][k];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gg = 0; gg < kWave / LPR; ++gg) packed = put_group(d[gg], gg, packed);
    }

    if (!active || !ok) return;
    if (ch.w < 0) {
        finish_store<VEC>(acc, ch.x, ch.z - ch.y, fo, f, C, ldc, epi, false);
    } else {
        store_vec<VEC>(partials + static_cast<int64_t>(ch.w) * ldp + fo, acc);
    }
}

// The output-resident passes (run_aggregate_resident).  One 1024-thread
// workgroup per CU owns rows [R0, R0 + nr) (nr <= kResidentRows) and keeps
// their running sums for one 32-column tile in LDS, while it walks the
// column blocks in order: all workgroups start together and have about the
// same work per block, so they gather from the same block's slice of B
// (rows_per_block x 128 bytes) at the same time and the slice stays in L2;
// the output is written once per tile, with the epilogue.  Within a block,
// the range's entries are contiguous in the blocked copy and are split
// evenly over the 128 lane groups (8 lanes x 4 columns each, as
// agg_sidx_kernel's), so heavy rows are shared and every batch of 16
// entries is full, across row boundaries.  A group walks its entries in
// order: a row that starts in its share is the group's ("owned"), summed
// as a chain continued from the row's LDS sum; the part of a row that
// started in an earlier group's share is summed from zero as a head
// partial.  After a barrier, the owner of a row that ran past the end of
// its share adds the later groups' heads of that row in group order.  The
// split depends on the structure alone, so the sums are deterministic.
struct ResidentArgs {
    const int32_t* brp;      // block s's row r at s * n + r
    const int32_t* wg_rows;  // the workgroups' first rows (gridDim.x + 1)
    const float* B;
    int64_t ldb;
    float* C;
    int64_t ldc;
    int64_t n;
    int64_t f;
    int64_t rows_per_block;
    int nb;
    // per phase (tile x block), the workgroups that finished it (zeroed
    // before the launch; null: no pacing)
    int* phase_count;
};

constexpr int kResGroups = kResidentThreads / 8;  // 8-lane groups of a workgroup
// Pacing: a workgroup starts phase q + 1 once every workgroup has finished
// phase q + 1 - kResSlack, so at most kResSlack blocks' slices are being
// gathered at a time.  The wait is bounded (kResSpin polls); after a
// time-out (workgroups not all resident) a workgroup stops waiting.  The
// pacing orders nothing: the sums do not depend on it.
constexpr int kResSlack = 2;
constexpr int kResSpin = 4096;

// TILED: B tile-major (rows of 128 bytes: offsets by shift); else
// row-major with a pitch of less than 2^16 bytes (24-bit multiplies).
template <bool TILED>
// (4 waves per SIMD: one workgroup per CU)
__global__ __launch_bounds__(kResidentThreads, 4) void agg_resident_kernel(
    ResidentArgs a, AggEpilogue epi) {
    constexpr int LPR = 8, VEC = 4, U = 16;
    __shared__ float4 sums[kResidentRows][LPR];
    __shared__ float4 heads[kResGroups][LPR];
    __shared__ int brps[kResidentRows + 1];
    __shared__ int head_row[kResGroups];  // -1: no head; -2: an empty share
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int R0 = a.wg_rows[blockIdx.x];
    const int nr = a.wg_rows[blockIdx.x + 1] - R0;
    const uint32_t pitch = static_cast<uint32_t>(a.ldb) * 4u;  // bytes per row of B
    // lane p of a group loads entries 2p and 2p + 1 of a batch (one dword)
    const uint32_t* cw = reinterpret_cast<const uint32_t*>(epi.ci16);
    const int ntiles = static_cast<int>((a.f + 31) / 32);
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    auto load_rows = [&](int s) {  // block s's row pointers of the range
        const int32_t* bp = a.brp + static_cast<int64_t>(s) * a.n + R0;
        for (int i = threadIdx.x; i <= nr; i += kResidentThreads) brps[i] = bp[i];
    };
    for (int i = threadIdx.x; i < nr * LPR; i += kResidentThreads) sums[i / LPR][i % LPR] = zero4;
    load_rows(0);
    __syncthreads();
    bool paced = true;  // (thread 0's)

    for (int q = 0; q < ntiles * a.nb; ++q) {
        const int tile = q / a.nb, s = q % a.nb;
        const int64_t fbase = static_cast<int64_t>(tile) * 32;
        const int64_t fo = fbase + static_cast<int64_t>(l) * VEC;
        const bool ok = fo < a.f;
        // block s's rows of the tile: a buffer range from the tile's first
        // column of the block's first row (the same for the whole
        // workgroup), and the lane's columns as an offset into each row
        // (lanes past f read the tile's first columns, unused)
        const int64_t row0 = static_cast<int64_t>(s) * a.rows_per_block;
        const int64_t rows_s = (a.n - row0 < a.rows_per_block ? a.n - row0 : a.rows_per_block);
        const float* bt = TILED ? a.B + static_cast<int64_t>(tile) * epi.b_tile_stride + row0 * 32
                                : a.B + row0 * a.ldb + fbase;
        const BufRsrc rsrc = buffer_rsrc(bt, static_cast<uint32_t>(rows_s * pitch));
        const uint32_t laneoff = ok ? static_cast<uint32_t>(l) * 16u : 0u;

        // the group's share [a0, b0) of the range's entries in block s
        const int E0 = brps[0], L = brps[nr] - E0;
        const int a0 = E0 + static_cast<int>((static_cast<int64_t>(g) * L) / kResGroups);
        const int b0 = E0 + static_cast<int>((static_cast<int64_t>(g + 1) * L) / kResGroups);
        const bool has = a0 < b0;
        // the row holding entry a0: the last r with brps[r] <= a0
        int r = 0;
        if (has) {
            int lo = 0, hi = nr;  // brps[lo] <= a0 < brps[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (brps[mid] <= a0) lo = mid;
                else hi = mid;
            }
            r = lo;
        }
        const int head_r = has && brps[r] < a0 ? r : -1;  // the share starts inside row r
        int end = has ? brps[r + 1] : 0;
        float acc[VEC] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (has && head_r < 0) {
            const float4 p4 = sums[r][l];
            acc[0] = p4.x;
            acc[1] = p4.y;
            acc[2] = p4.z;
            acc[3] = p4.w;
        }
        float hacc[VEC] = {0.0f, 0.0f, 0.0f, 0.0f};

        // 16-entry batches from the dword-aligned start of the share
        const int p0 = a0 & ~1;
        const int nbt = has ? (b0 - p0 + 15) >> 4 : 0;
        int nmax = 0;
#pragma unroll
        for (int gg = 0; gg < kWave / LPR; ++gg) {
            const int x = __builtin_amdgcn_readlane(nbt, gg * LPR);
            nmax = x > nmax ? x : nmax;
        }
        // dword offset of batch t (the last batch once done; 0 without any):
        // every load stays within the share's batches, at most 15 entries
        // past its end (the blocked copy keeps 64 bytes of padding)
        auto batch_off = [&](int t) { return nbt > 0 ? (p0 >> 1) + 8 * (t < nbt ? t : nbt - 1) : 0; };
        uint32_t packed = cw[batch_off(0) + l];

        // where the current row ends, while that is inside the share (else
        // never: -1)
        int endv = has && end < b0 ? end : -1;
        for (int t = 0; t < nmax; ++t) {
            const int base = p0 + 16 * t;
            const int lo = a0 - base, cnt = b0 - base;  // slots [lo, cnt) are the share's
            // the lane's two slots 2l and 2l + 1: outside the share, column
            // 0xFFFF, past the range (at most 65535 rows): they gather zeros
            const uint32_t keep = (2 * l >= lo && 2 * l < cnt ? 0x0000FFFFu : 0u) |
                                  (2 * l + 1 >= lo && 2 * l + 1 < cnt ? 0xFFFF0000u : 0u);
            const uint32_t pk = (packed & keep) | ~keep;
            const uint32_t c0 = pk & 0xFFFFu, c1 = pk >> 16;
            Float4v bv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t col = static_cast<uint32_t>(__shfl((u & 1) ? c1 : c0, u >> 1, LPR));
                const uint32_t off = TILED ? (col << 7) + laneoff : __umul24(col, pitch) + laneoff;
                bv[u] = raw_buffer_load_f32x4(rsrc, off, 0u, 0);
            }
            // the next batch's indices, behind this batch's gathers
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t next = cw[batch_off(t + 1) + l];
            __builtin_amdgcn_sched_barrier(0);
            int dend = endv - base;  // the slot where the current row ends (if in 0..15)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (dend == u) {
                    // row r ends before this entry: keep its sum, move on to
                    // the row holding the entry (past rows without entries)
                    if (r == head_r) {
#pragma unroll
                        for (int k = 0; k < VEC; ++k) hacc[k] = acc[k];
                    } else {
                        sums[r][l] = make_float4(acc[0], acc[1], acc[2], acc[3]);
                    }
                    int r2 = r + 1;
                    while (brps[r2 + 1] == end) ++r2;
                    r = r2;
                    end = brps[r2 + 1];
                    endv = end < b0 ? end : -1;
                    dend = endv - base;
                    const float4 p4 = sums[r2][l];
                    acc[0] = p4.x;
                    acc[1] = p4.y;
                    acc[2] = p4.z;
                    acc[3] = p4.w;
                }
                // (slots outside the share add zeros)
                acc[0] += bv[u].x;
                acc[1] += bv[u].y;
                acc[2] += bv[u].z;
                acc[3] += bv[u].w;
            }
            packed = next;
        }

        // the share's last row: a head (the share lies inside it) or owned;
        // an owned row that runs past the share's end collects the heads
        int tail = -1;
        if (has) {
            if (r == head_r) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) hacc[k] = acc[k];
            } else {
                sums[r][l] = make_float4(acc[0], acc[1], acc[2], acc[3]);
                if (end > b0) tail = r;
            }
        }
        heads[g][l] = make_float4(hacc[0], hacc[1], hacc[2], hacc[3]);
        if (l == 0) head_row[g] = has ? head_r : -2;
        __syncthreads();
        if (tail >= 0) {
            const float4 p4 = sums[tail][l];
            float x[VEC] = {p4.x, p4.y, p4.z, p4.w};
            for (int g2 = g + 1; g2 < kResGroups; ++g2) {
                const int hr = head_row[g2];
                if (hr == -2) continue;  // an empty share
                if (hr != tail) break;
                const float4 h4 = heads[g2][l];
                x[0] += h4.x;
                x[1] += h4.y;
                x[2] += h4.z;
                x[3] += h4.w;
            }
            sums[tail][l] = make_float4(x[0], x[1], x[2], x[3]);
        }
        if (s == a.nb - 1) {
            // the tile is complete: store it with the epilogue
            __syncthreads();
            if (ok) {
                for (int rr = g; rr < nr; rr += kResGroups) {
                    const float4 p4 = sums[rr][l];
                    float x[VEC] = {p4.x, p4.y, p4.z, p4.w};
                    finish_store<VEC>(x, R0 + rr, 0, fo, a.f, a.C, a.ldc, epi, false);
                }
            }
            __syncthreads();
            if (q + 1 < ntiles * a.nb)
                for (int i = threadIdx.x; i < nr * LPR; i += kResidentThreads) sums[i / LPR][i % LPR] = zero4;
        }
        if (q + 1 < ntiles * a.nb) load_rows((q + 1) % a.nb);
        if (threadIdx.x == 0 && a.phase_count != nullptr) {
            atomicAdd(a.phase_count + q, 1);
            const int wait_q = q + 1 - kResSlack;
            if (paced && q + 1 < ntiles * a.nb && wait_q >= 0) {
                int it = 0;
                while (__hip_atomic_load(a.phase_count + wait_q, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) < static_cast<int>(gridDim.x)) {
                    if (++it == kResSpin) {
                        paced = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
        }
        __syncthreads();
    }
}

// Finishes split rows: partials of a row are combined in chunk order.
template <int VEC, int LPR, int VPL, int MODE>
__global__ __launch_bounds__(256) void agg_reduce_kernel(const int4* __restrict__ split,
                                                         int64_t n_split,
                                                         const int64_t* __restrict__ n_split_dev,
                                                         const float* __restrict__ partials,
                                                         int64_t ldp, float* __restrict__ C,
                                                         int64_t ldc, int64_t f,
                                                         AggEpilogue epi) {
    constexpr int GPB = 256 / LPR;
    constexpr int TILE = LPR * VPL * VEC;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t sid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (sid >= (n_split_dev ? *n_split_dev : n_split)) return;
    const int4 sp = split[sid];
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        const int64_t fo = fbase + static_cast<int64_t>(l + v * LPR) * VEC;
        if (fo >= f) continue;
        float acc[VEC];
        load_vec<VEC>(partials + static_cast<int64_t>(sp.y) * ldp + fo, acc);
        for (int c = 1; c < sp.z; ++c) {
            float t[VEC];
            load_vec<VEC>(partials + static_cast<int64_t>(sp.y + c) * ldp + fo, t);
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                acc[k] = MODE == kAggMax ? ((acc[k] < t[k]) ? t[k] : acc[k]) : acc[k] + t[k];
        }
        finish_store<VEC>(acc, sp.x, sp.w, fo, f, C, ldc, epi, epi.acc != 0);
    }
}

// Column tile of the long-row kernel: the lane groups' tile when they are
// given (column-blocked passes), else 32, 64 or 128 columns by f.
inline int long_tile(int64_t f, const LaneLayout& L) {
    if (L.tile == 32 || L.tile == 64 || L.tile == 128) {
        if (L.n_tiles > 1 || L.tile >= f) return L.tile;
    }
    return f <= 32 ? 32 : f <= 64 ? 64 : 128;
}

// Rows of more than one chunk summed as ONE chain each, in nonzero order:
// acc = combine(acc, B[col_e, j], w_e) for e along the row, exactly the
// reference's loop (ops.cpp:266-287 for SpMM).  One workgroup takes one
// (row, TW-column tile).  A chain is serial, so what bounds a long row is
// how many of its gathers are in flight; here all 256 threads issue them:
// G = TW / VEC lanes fetch one entry's tile row, 256 / G entries per round,
// U rounds per batch (32 floats in flight per thread), BE = 8192 / TW
// entries per batch, landing in LDS.  Threads [0, TW) then walk the batch
// in order, one column each, while the next two batches' gathers are in
// flight (two register sets, two 32 KB LDS buffers, one barrier per
// batch).  The row's column indices go through LDS (one coalesced load per
// entry), its weights likewise.  Split rows come longest first, so the
// longest chains start first.
template <int VEC, int TW, int MODE>
__global__ __launch_bounds__(256, 2) void agg_long_kernel(
    const int4* __restrict__ split, int64_t n_split, const int64_t* __restrict__ n_split_dev,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ ci,
    const float* __restrict__ av, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, int64_t f, AggEpilogue epi) {
    static_assert(MODE == kAggWeighted || MODE == kAggSum || MODE == kAggSumTail ||
                      MODE == kAggMax,
                  "long rows: weighted, sum or max");
    static_assert(TW == 32 || TW == 64 || TW == 128, "tile width");
    constexpr int G = TW / VEC;   // lanes per gathered entry
    constexpr int R = 256 / G;    // entries per round
    constexpr int U = 32 / VEC;   // rounds per batch
    constexpr int BE = U * R;     // entries per batch
    static_assert(BE * TW == 8192 && BE <= 256, "batch shape");
    __shared__ __align__(16) float dbuf[2][BE * TW];
    __shared__ float wbuf[2][BE];
    __shared__ int cbuf[2][BE];

    const int64_t sid = blockIdx.x;
    if (sid >= (n_split_dev ? *n_split_dev : n_split)) return;  // uniform
    const int4 sp = split[sid];
    const int row = sp.x;
    const int rb = row_ptr[row];
    const int re = rb + sp.w;
    const int nb = (sp.w + BE - 1) / BE;
    const int tid = threadIdx.x;
    const int q = tid / G, p = tid % G;
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TW;
    const int64_t fo = fbase + static_cast<int64_t>(p) * VEC;
    // lanes past f load the tile's first vector (in bounds), never used
    const int64_t fl = fo < f ? fo : fbase;
    const char* bl = reinterpret_cast<const char*>(
        epi.b_tile_stride > 0 ? B + (fl >> 5) * epi.b_tile_stride + (fl & 31) : B + fl);
    const uint32_t pitch = static_cast<uint32_t>(ldb) * 4u;

    // Entry tid of batch t (its index clamped into the row, so every load is
    // in bounds and unconditional: the slots past the row's end fetch a real
    // entry whose value is never used, and no load needs a default value, so
    // no wait on earlier loads is forced).  Only threads below BE store them.
    const bool c16 = epi.ci16 != nullptr;
    auto entry = [&](int t) {
        const int64_t idx = static_cast<int64_t>(rb) + static_cast<int64_t>(t) * BE + tid;
        return idx < re ? static_cast<int>(idx) : re - 1;
    };
    auto col_of = [&](int t) -> int {
        const int idx = entry(t);
        return c16 ? static_cast<int>(epi.ci16[idx]) : ci[idx];
    };
    auto w_of = [&](int t) -> float {
        if constexpr (MODE == kAggWeighted) return av[entry(t)];
        return 1.0f;
    };
    // two register sets: the gathers of batches t + 1 and t + 2 are in flight
    // while batch t's chains run
    float g0[U][VEC], g1[U][VEC];
    // gathers of batch t (columns from cbuf[t & 1]) into g: every slot,
    // those past the row's end included (their columns are real ones); a
    // batch past the row's last (the steps run in pairs) loads row 0 only
    auto issue = [&](int t, float (&g)[U][VEC]) {
        const uint32_t pm = t < nb ? pitch : 0u;
        int col[U];
#pragma unroll
        for (int u = 0; u < U; ++u) col[u] = cbuf[t & 1][u * R + q];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(col[u])) * pm;
            load_vec<VEC>(reinterpret_cast<const float*>(bl + off), g[u]);
        }
    };
    auto land = [&](int t, const float (&g)[U][VEC]) {
#pragma unroll
        for (int u = 0; u < U; ++u) store_vec<VEC>(&dbuf[t & 1][(u * R + q) * TW + p * VEC], g[u]);
    };

    // chain lane: column fj of the tile; a blocked pass after the first
    // continues the row's chain from the value the earlier passes stored
    const int64_t fj = fbase + tid;
    const bool chain_lane = tid < TW;
    float acc = MODE == kAggMax ? -INFINITY : 0.0f;
    if (epi.acc && chain_lane && fj < f) acc = C[static_cast<int64_t>(row) * ldc + fj];
    auto walk = [&](int t) {
        if (!chain_lane) return;
        const float* d = &dbuf[t & 1][tid];
        const float* w = wbuf[t & 1];
        const int cnt = re - rb - t * BE;
        if (cnt >= BE) {
            // a full batch, unrolled: the LDS reads are scheduled ahead of
            // the chain's fmas
#pragma unroll
            for (int e = 0; e < BE; ++e) acc = combine<MODE>(acc, d[e * TW], w[e]);
        } else {
            int e = 0;
            for (; e + 8 <= cnt; e += 8) {
#pragma unroll
                for (int k = 0; k < 8; ++k) acc = combine<MODE>(acc, d[(e + k) * TW], w[e + k]);
            }
            for (; e < cnt; ++e) acc = combine<MODE>(acc, d[e * TW], w[e]);
        }
    };

    // Batch x's columns sit in cbuf[x & 1] until its gathers are issued, its
    // weights in wbuf[x & 1] and its rows in dbuf[x & 1] while it is walked.
    // Step t (after a barrier: batch t landed, batch t + 1 in flight in the
    // other register set, batch t + 2's columns in cbuf): issue batch t + 2,
    // walk batch t, land batch t + 1 with its weights, store batch t + 3's
    // columns, barrier.
    const bool meta = tid < BE;  // threads that store columns and weights
    {
        const int c0 = col_of(0);
        const float w0 = w_of(0);
        const int c1 = col_of(1);
        if (meta) {
            cbuf[0][tid] = c0;
            wbuf[0][tid] = w0;
            cbuf[1][tid] = c1;
        }
    }
    __syncthreads();
    // weights of the batches in flight, one register per set like the
    // gathers (a copy between registers would wait for the load); in a
    // step the next columns and weights are loaded before the gathers, so
    // storing them waits for those loads only, not for the gathers
    float wa = 0.0f;
    float wb = w_of(1);
    issue(0, g0);
    issue(1, g1);
    const int c2 = col_of(2);
    __syncthreads();  // cbuf[0] read by every issue(0)
    land(0, g0);
    if (meta) cbuf[0][tid] = c2;
    __syncthreads();
    auto step = [&](int t, float (&gnext)[U][VEC], float (&gland)[U][VEC], float& wnext,
                    const float& wland) {
        // gnext / wnext: the sets free since batch t landed; gland / wland:
        // batch t + 1's
        // Every load and store of a step is unconditional, so that the wait
        // counters see one path: a branch around a register set's loads
        // would make the compiler wait, at its next use, for every load
        // issued since -- the gathers in flight included.  Past the row's
        // end the loads fetch real entries or row 0 (all in bounds), and the
        // stores rewrite buffers that are not read again.
        const int c3 = col_of(t + 3);
        wnext = w_of(t + 2);
        issue(t + 2, gnext);
        walk(t);
        land(t + 1, gland);
        if (meta) {
            wbuf[(t + 1) & 1][tid] = wland;
            cbuf[(t + 1) & 1][tid] = c3;
        }
        __syncthreads();
    };
    // steps in pairs (the register sets alternate); an odd nb ends with one
    // step past the row, which walks nothing
    for (int t = 0; t < nb; t += 2) {
        step(t, g0, g1, wa, wb);
        step(t + 1, g1, g0, wb, wa);
    }
    if (chain_lane && fj < f) {
        float x[1] = {acc};
        finish_store<1>(x, row, sp.w, fj, f, C, ldc, epi, false);
    }
}

template <int VEC, int MODE>
void launch_long(const PlanView& p, int tw, int64_t f, const int32_t* ci, const float* av,
                 const float* B, int64_t ldb, float* C, int64_t ldc, const AggEpilogue& epi,
                 hipStream_t s) {
    require(p.row_ptr != nullptr, "aggregate: long rows need the plan's row pointers");
    const int64_t* dc = p.dev_counts ? p.dev_counts + 1 : nullptr;
    const dim3 grid(static_cast<unsigned>(p.n_split), static_cast<unsigned>(ceil_div(f, tw)));
#define TG_LONG(TW_)                                                                     \
    if (tw == TW_) {                                                                     \
        agg_long_kernel<VEC, TW_, MODE><<<grid, 256, 0, s>>>(                            \
            p.split, p.n_split, dc, p.row_ptr, ci, av, B, ldb, C, ldc, f, epi);          \
        TG_LAUNCH_CHECK();                                                               \
        return;                                                                          \
    }
    TG_LONG(32)
    TG_LONG(64)
    TG_LONG(128)
#undef TG_LONG
    throw std::logic_error("aggregate: no long-row kernel for this tile width");
}

template <int VEC, int LPR, int VPL, int MODE>
void launch_agg(const PlanView& p, const LaneLayout& L, int64_t f, const int32_t* ci,
                const float* av, const float* B, int64_t ldb, float* C, int64_t ldc,
                const AggEpilogue& epi, hipStream_t s) {
    constexpr int GPB = 256 / LPR;
    const int64_t ldp = round_up(f, VEC);  // padded partial rows
    const int64_t* dc = p.dev_counts;
    if (epi.long_rows && p.n_split > 0) {
        // the longest chains first; the chunk kernel then skips their chunks
        if constexpr (MODE == kAggAttn) {
            throw std::logic_error("aggregate: long rows do not take attention weights");
        } else {
            launch_long<VEC, MODE>(p, long_tile(f, L), f, ci, av, B, ldb, C, ldc, epi, s);
        }
    }
    if (p.n_chunks > 0) {
        // grid.y = column tile: the workgroups resident at a time (dispatched
        // in x order) gather from one or two tiles of B
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_chunks, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        agg_chunk_kernel<VEC, LPR, VPL, MODE><<<grid, 256, 0, s>>>(
            p.chunks, p.n_chunks, dc, ci, av, B, ldb, C, ldc, p.partials, ldp, f, epi);
        TG_LAUNCH_CHECK();
    }
    if (p.n_split > 0 && !epi.long_rows) {
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_split, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        agg_reduce_kernel<VEC, LPR, VPL, MODE><<<grid, 256, 0, s>>>(
            p.split, p.n_split, dc ? dc + 1 : nullptr, p.partials, ldp, C, ldc, f, epi);
        TG_LAUNCH_CHECK();
    }
}

// The fast column-blocked passes over 16-bit indices (agg_sidx_kernel), then
// split rows as launch_agg<4, 8, 1, kAggSumTail>'s.
void launch_agg_sidx(const PlanView& p, const LaneLayout& L, int64_t f, const float* B,
                     int64_t ldb, float* C, int64_t ldc, const AggEpilogue& epi, hipStream_t s) {
    constexpr int GPB = 256 / 8;
    const int64_t ldp = round_up(f, 4);
    const int64_t* dc = p.dev_counts;
    if (epi.long_rows && p.n_split > 0)
        launch_long<4, kAggSumTail>(p, long_tile(f, L), f, nullptr, nullptr, B, ldb, C, ldc,
                                    epi, s);
    if (p.n_chunks > 0) {
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_chunks, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        // buffer gathers where column 0xFFFF lies past B's rows (blocks of
        // at most 65535 rows) and a row's offsets fit 32 bits
        const bool tiled = epi.b_tile_stride > 0;
        const bool buf = epi.b_rows > 0 && (tiled ? ldb == 32 : ldb < 16384) &&
                         reinterpret_cast<uintptr_t>(B) % 16 == 0;
        if (buf && tiled)
            agg_sidx_kernel<1><<<grid, 256, 0, s>>>(p.chunks, p.n_chunks, dc, B, ldb, C, ldc,
                                                    p.partials, ldp, f, epi);
        else if (buf)
            agg_sidx_kernel<2><<<grid, 256, 0, s>>>(p.chunks, p.n_chunks, dc, B, ldb, C, ldc,
                                                    p.partials, ldp, f, epi);
        else
            agg_sidx_kernel<0><<<grid, 256, 0, s>>>(p.chunks, p.n_chunks, dc, B, ldb, C, ldc,
                                                    p.partials, ldp, f, epi);
        TG_LAUNCH_CHECK();
    }
    if (p.n_split > 0 && !epi.long_rows) {
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_split, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        agg_reduce_kernel<4, 8, 1, kAggSumTail><<<grid, 256, 0, s>>>(
            p.split, p.n_split, dc ? dc + 1 : nullptr, p.partials, ldp, C, ldc, f, epi);
        TG_LAUNCH_CHECK();
    }
}

template <int VEC, int MODE>
void dispatch_lpr(const PlanView& p, const LaneLayout& L, int64_t f, const int32_t* ci,
                  const float* av, const float* B, int64_t ldb, float* C, int64_t ldc,
                  const AggEpilogue& epi, hipStream_t s) {
#define TG_AGG_CASE(LPR_, VPL_)                                                          \
    if (L.lpr == LPR_ && L.vpl == VPL_)                                                  \
        return launch_agg<VEC, LPR_, VPL_, MODE>(p, L, f, ci, av, B, ldb, C, ldc, epi, s);
    TG_AGG_CASE(4, 1)
    TG_AGG_CASE(8, 1)
    TG_AGG_CASE(16, 1)
    TG_AGG_CASE(32, 1)
    TG_AGG_CASE(64, 1)
#undef TG_AGG_CASE
    throw std::logic_error("aggregate: no kernel for this lane layout");
}

}  // namespace

void run_aggregate(const tg_spmm_plan_s& p, int64_t f, const int32_t* ci, const float* av,
                   const float* B, int64_t ldb, float* C, int64_t ldc, const AggEpilogue& epi,
                   hipStream_t s, int tile_cols) {
    run_aggregate(plan_view(p), f, ci, av, B, ldb, C, ldc, epi, s, tile_cols);
}

void run_aggregate(const PlanView& p, int64_t f, const int32_t* ci, const float* av,
                   const float* B, int64_t ldb, float* C, int64_t ldc, const AggEpilogue& epi,
                   hipStream_t s, int tile_cols) {
    if (p.m == 0 || f == 0) return;
    const bool tiled_b = epi.b_tile_stride > 0;
    require(!tiled_b || ((tile_cols == 32 || tile_cols == 64) && ldb == 32),
            "aggregate: a tile-major B needs 32- or 64-column groups and tiles of pitch 32");
    require((tiled_b || ldb >= f) && ldc >= f, "aggregate: leading dimension smaller than f");
    require(ldb < (int64_t(1) << 30), "aggregate: B's leading dimension must be < 2^30");
    require(epi.self == nullptr || (epi.self_tile_stride > 0 ? epi.ld_self == 32
                                                              : epi.ld_self >= f),
            "aggregate: self ld smaller than f");
    if (p.n_split > 0)
        require(f <= p.max_f,
                "aggregate: feature width " + std::to_string(f) +
                    " exceeds the plan's max_f " + std::to_string(p.max_f));
    // Loads use the widest access the rows of B allow (a padded leading
    // dimension lets the last vector of a row run into the padding); stores
    // and the epilogue operands are vectors only when they are aligned too.
    const int vec = tiled_b ? pick_vec(32, {epi.b_tile_stride}, {B}) : pick_load_vec(f, ldb, B);
    AggEpilogue e = epi;
    e.vec_io = pick_vec(f, {ldc, epi.self ? epi.ld_self : vec}, {C, epi.self, epi.bias}) >= vec;
    require(tile_cols == 0 || tile_cols == 32 || tile_cols == 64,
            "aggregate: tile_cols must be 0, 32 or 64");
    LaneLayout L = choose_layout(f, vec);
    if (tile_cols > 0) {
        L.lpr = tile_cols / vec;
        L.vpl = 1;
        L.tile = tile_cols;
        L.n_tiles = static_cast<int>(ceil_div(f, tile_cols));
    }
#define TG_AGG_MODE(M_)                                                                \
    if (vec == 4) return dispatch_lpr<4, M_>(p, L, f, ci, av, B, ldb, C, ldc, e, s);      \
    if (vec == 2) return dispatch_lpr<2, M_>(p, L, f, ci, av, B, ldb, C, ldc, e, s);      \
    return dispatch_lpr<1, M_>(p, L, f, ci, av, B, ldb, C, ldc, e, s);
    if (epi.max) {
        require(!epi.mean, "aggregate: max and mean are exclusive");
        TG_AGG_MODE(kAggMax)
    }
    if (epi.att_dst) {
        require(!av && !epi.mean && epi.w_head_cols >= 1 &&
                    (epi.w_head_cols >= f || epi.w_head_cols % L.tile == 0),
                "aggregate: attention weights need whole column tiles per head");
        TG_AGG_MODE(kAggAttn)
    }
    if (av) {
        TG_AGG_MODE(kAggWeighted)
    }
    if (epi.mask_tail && vec == 4 && L.lpr == 8 && L.vpl == 1) {  // the 32-column passes only
        // 16-bit indices are a blocked copy's, padded for the scalar loads
        if (epi.ci16) return launch_agg_sidx(p, L, f, B, ldb, C, ldc, e, s);
        return launch_agg<4, 8, 1, kAggSumTail>(p, L, f, ci, av, B, ldb, C, ldc, e, s);
    }
    TG_AGG_MODE(kAggSum)
#undef TG_AGG_MODE
}

bool resident_ok(const BlockedCSR& bk, int64_t f, const float* B, int64_t ldb,
                 const AggEpilogue& epi) {
    // (column 0xFFFF must lie past every block: at most 65535 rows per block)
    if (bk.resident_wgs <= 0 || !bk.idx16 || bk.weighted || bk.group_cols != 32 ||
        bk.rows_per_block > 65535)
        return false;
    if (epi.max || epi.att_dst || f <= 0) return false;
    const bool tiled = epi.b_tile_stride > 0;
    if (tiled) return ldb == 32 && epi.b_tile_stride % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(B) % 16 == 0;
    // row-major: rows of less than 2^16 bytes (24-bit offsets)
    return ldb % 4 == 0 && ldb >= round_up(f, 4) && ldb < 16384 &&
           reinterpret_cast<uintptr_t>(B) % 16 == 0;
}

void run_aggregate_resident(const BlockedCSR& bk, int64_t f, const float* B, int64_t ldb,
                            float* C, int64_t ldc, const AggEpilogue& epi, hipStream_t s) {
    require(resident_ok(bk, f, B, ldb, epi), "resident aggregation: unsupported pass");
    require(!epi.acc && !epi.skip_empty, "resident aggregation: pass flags are internal");
    require(ldc >= f, "aggregate: leading dimension smaller than f");
    require(epi.self == nullptr || (epi.self_tile_stride > 0 ? epi.ld_self == 32
                                                              : epi.ld_self >= f),
            "aggregate: self ld smaller than f");
    if (bk.n == 0 || f == 0) return;
    AggEpilogue e = epi;
    e.ci16 = bk.bci.as<uint16_t>();
    if (e.mean) e.deg_rp = bk.rp;
    e.vec_io = pick_vec(f, {ldc, epi.self ? epi.ld_self : 4}, {C, epi.self, epi.bias}) >= 4;
    ResidentArgs a{};
    a.brp = bk.brp.as<int32_t>();
    a.wg_rows = bk.wg_rows.as<int32_t>();
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.n = bk.n;
    a.f = f;
    a.rows_per_block = bk.rows_per_block;
    a.nb = static_cast<int>(bk.n_blocks);
    const int64_t phases = ceil_div(f, 32) * bk.n_blocks;
    if (phases <= bk.max_phases) {
        a.phase_count = bk.phase_count.as<int>();
        fill_i32(a.phase_count, phases, 0, s);
    }
    if (epi.b_tile_stride > 0)
        agg_resident_kernel<true>
            <<<static_cast<unsigned>(bk.resident_wgs), kResidentThreads, 0, s>>>(a, e);
    else
        agg_resident_kernel<false>
            <<<static_cast<unsigned>(bk.resident_wgs), kResidentThreads, 0, s>>>(a, e);
    TG_LAUNCH_CHECK();
}

}  // namespace tg

// ---------------------------------------------------------------------------
// SpMM without allocation (tg_spmm_noalloc, whose C-ABI and fixed device
// array are in noalloc.hip): the plan of one call -- its build temporaries,
// chunks, split records and partials -- carved from a caller-given device
// array instead of allocated buffers.  The host never reads the plan's
// counts: the grids cover upper bounds and the kernels read the true counts
// from the array, so the call only enqueues kernels.
// ---------------------------------------------------------------------------
namespace tg {
namespace {

// Capacities of a plan for m rows and nnz nonzeros in chunks of c:
// chunks <= m + nnz / c (each row one chunk, plus one per further c
// entries); split rows hold more than c entries, so there are at most
// nnz / (c + 1) of them; their partial slots number ceil(deg / c) <= 1 +
// deg / c each, at most n_split + nnz / c.
struct NoAllocPlan {
    int64_t cap_chunks = 0, cap_split = 0, cap_partials = 0;
    PlanTemps t{};
    int4* chunks = nullptr;
    int4* split = nullptr;
    float* partials = nullptr;
};

NoAllocPlan carve_noalloc(Carver& cv, int64_t m, int64_t nnz, int64_t f) {
    const int64_t c = kDefaultChunk;
    NoAllocPlan P;
    P.cap_chunks = m + nnz / c;
    P.cap_split = std::min(m, nnz / (c + 1));
    P.cap_partials = P.cap_split > 0 ? P.cap_split + nnz / c : 0;
    P.t = carve_temps(cv, m);
    P.chunks = cv.take<int4>(static_cast<size_t>(P.cap_chunks));
    P.split = cv.take<int4>(static_cast<size_t>(std::max<int64_t>(P.cap_split, 1)));
    P.partials = cv.take<float>(static_cast<size_t>(P.cap_partials * round_up(f, 4)));
    return P;
}

// A row_ptr whose last entry exceeds the caller's nnz overflows the plan's
// capacities; plan_bins_kernel then zeroes the counts (nothing else runs)
// and sets totals[3], and this kernel fills C with NaN, so that the misuse
// shows in the output instead of leaving it unwritten.
__global__ __launch_bounds__(256) void noalloc_poison_kernel(const int64_t* __restrict__ totals,
                                                             float* __restrict__ c, int64_t m,
                                                             int64_t f, int64_t ldc) {
    if (totals[3] == 0) return;
    const int64_t n = m * f;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        c[(i / f) * ldc + i % f] = __builtin_nanf("");
}

}  // namespace

size_t spmm_noalloc_bytes(int64_t m, int64_t nnz, int64_t f) {
    Carver sizing(nullptr, 0);
    carve_noalloc(sizing, m, nnz, f);
    return sizing.bytes();
}

void spmm_noalloc(char* scratch, size_t scratch_bytes, int64_t m, int64_t f, int64_t nnz,
                  const int32_t* rp, const int32_t* ci, const float* v, const float* b,
                  int64_t ldb, float* c, int64_t ldc, hipStream_t s) {
    Carver cv(scratch, scratch_bytes);
    const NoAllocPlan P = carve_noalloc(cv, m, nnz, f);
    const int chunk = static_cast<int>(kDefaultChunk);
    const unsigned nblk = static_cast<unsigned>(ceil_div(m, 256));
    fill_i32(P.t.bin_count, 2 * kPlanBins, 0, s);  // a kernel, so the call stays capturable
    plan_count_kernel<<<nblk, 256, 0, s>>>(rp, m, chunk, P.t.split_cnt, P.t.is_split,
                                           P.t.bin_count);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(P.t.split_cnt, P.t.slot_base, m, P.t.scan_tmp, s);
    exclusive_scan_i32(P.t.is_split, P.t.split_pos, m, P.t.scan_tmp, s);
    plan_bins_kernel<<<1, 64, 0, s>>>(P.t.bin_count, P.t.bin_cursor, P.t.slot_base,
                                      P.t.split_pos, m, P.t.totals, P.cap_chunks, P.cap_split,
                                      P.cap_partials);
    TG_LAUNCH_CHECK();
    plan_scatter_kernel<<<nblk, 256, 0, s>>>(rp, m, chunk, P.t.slot_base, P.t.bin_cursor,
                                             P.chunks, P.split, P.cap_chunks, P.cap_split);
    TG_LAUNCH_CHECK();
    PlanView pv;
    pv.m = m;
    pv.max_f = f;
    pv.n_chunks = P.cap_chunks;
    pv.n_split = P.cap_split;
    pv.chunks = P.chunks;
    pv.split = P.split;
    pv.partials = P.partials;
    pv.row_ptr = rp;
    pv.dev_counts = P.t.totals;  // [0] chunks, [1] split rows
    AggEpilogue epi;
    epi.long_rows = 1;  // tg_spmm's order: every row one chain in nonzero order
    run_aggregate(pv, f, ci, v, b, ldb, c, ldc, epi, s);
    const unsigned pblk = static_cast<unsigned>(std::min<int64_t>(ceil_div(m * f, 256), 1024));
    noalloc_poison_kernel<<<pblk, 256, 0, s>>>(P.t.totals, c, m, f, ldc);
    TG_LAUNCH_CHECK();
}

}  // namespace tg

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
using tg::guard;
using tg::require;

extern "C" {

int tg_spmm_plan_create(int64_t m, int64_t nnz_bound, const int32_t* row_ptr, int64_t max_f,
                        int64_t chunk_nnz, tg_stream_t stream, tg_spmm_plan_t* plan_out) {
    return guard([&] {
        require(plan_out != nullptr, "tg_spmm_plan_create: plan_out is null");
        auto p = std::make_unique<tg_spmm_plan_s>();
        tg::build_plan(*p, m, nnz_bound, row_ptr, max_f, chunk_nnz,
                       static_cast<hipStream_t>(stream));
        *plan_out = p.release();
    });
}

int tg_spmm_plan_destroy(tg_spmm_plan_t plan) {
    return guard([&] { delete plan; });
}

int tg_spmm_plan_info(tg_spmm_plan_t plan, int64_t* n_chunks, int64_t* n_split_rows,
                      int64_t* n_partials) {
    return guard([&] {
        require(plan != nullptr, "tg_spmm_plan_info: plan is null");
        if (n_chunks) *n_chunks = plan->n_chunks;
        if (n_split_rows) *n_split_rows = plan->n_split;
        if (n_partials) *n_partials = plan->n_partials;
    });
}

int tg_spmm_plan_set_precision(tg_spmm_plan_t plan, int precision) {
    return guard([&] {
        require(plan != nullptr, "tg_spmm_plan_set_precision: plan is null");
        require(precision == TG_PRECISION_FAST || precision == TG_PRECISION_EXACT,
                "tg_spmm_plan_set_precision: precision must be TG_PRECISION_FAST or "
                "TG_PRECISION_EXACT");
        plan->precision = precision;
    });
}

int tg_spmm_execute(tg_spmm_plan_t plan, int64_t k, int64_t f, const int32_t* row_ptr,
                    const int32_t* col_ind, const float* val, const float* b, int64_t ldb,
                    float* c, int64_t ldc, tg_stream_t stream) {
    return guard([&] {
        require(plan != nullptr, "tg_spmm_execute: plan is null");
        require(row_ptr == plan->row_ptr,
                "tg_spmm_execute: row_ptr differs from the one the plan was built for");
        require(k >= 0 && f >= 0, "spmm: negative dimension");
        require(val != nullptr, "spmm: val is null");
        tg::AggEpilogue epi;
        epi.long_rows = plan->precision == TG_PRECISION_EXACT;
        tg::run_aggregate(*plan, f, col_ind, val, b, ldb, c, ldc, epi,
                          static_cast<hipStream_t>(stream));
    });
}

int tg_spmm_execute_epilogue(tg_spmm_plan_t plan, int64_t k, int64_t f, const int32_t* row_ptr,
                             const int32_t* col_ind, const float* val, const float* b,
                             int64_t ldb, float* c, int64_t ldc, const float* bias, int epilogue,
                             tg_stream_t stream) {
    return guard([&] {
        require(plan != nullptr, "tg_spmm_execute_epilogue: plan is null");
        require(row_ptr == plan->row_ptr,
                "tg_spmm_execute_epilogue: row_ptr differs from the one the plan was built for");
        require(k >= 0 && f >= 0, "spmm: negative dimension");
        require(val != nullptr, "spmm: val is null");
        require(epilogue == TG_EPI_NONE || epilogue == TG_EPI_RELU || epilogue == TG_EPI_ELU,
                "tg_spmm_execute_epilogue: unknown epilogue");
        tg::AggEpilogue epi;
        epi.long_rows = plan->precision == TG_PRECISION_EXACT;
        epi.bias = bias;
        // add_bias (ops.cpp:622-661), then relu_inplace / elu_inplace with
        // alpha 1 (ops.cpp:328-392): the same operations in the store
        epi.act = epilogue == TG_EPI_RELU ? TG_ACT_RELU : TG_ACT_NONE;
        epi.post = epilogue == TG_EPI_ELU ? TG_POST_ELU : TG_POST_NONE;
        tg::run_aggregate(*plan, f, col_ind, val, b, ldb, c, ldc, epi,
                          static_cast<hipStream_t>(stream));
    });
}

int tg_spmm_ex(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
               const int32_t* col_ind, const float* val, const float* b, int64_t ldb, float* c,
               int64_t ldc, int precision, tg_stream_t stream) {
    return guard([&] {
        require(m >= 0 && k >= 0 && f >= 0 && nnz >= 0, "spmm: negative dimension");
        require(precision == TG_PRECISION_FAST || precision == TG_PRECISION_EXACT,
                "spmm: precision must be TG_PRECISION_FAST or TG_PRECISION_EXACT");
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (m == 0 || f == 0) return;
        if (nnz == 0) {
            // ops.cpp:231-236: the result is the zero-initialised C.
            tg::fill_zero_2d(c, m, f, ldc, s);
            return;
        }
        tg_spmm_plan_s p;
        tg::build_plan(p, m, nnz, row_ptr, f, 0, s);
        tg::AggEpilogue epi;
        epi.long_rows = precision == TG_PRECISION_EXACT;
        tg::run_aggregate(p, f, col_ind, val, b, ldb, c, ldc, epi, s);
        TG_HIP(hipStreamSynchronize(s));  // the plan's buffers are freed on return
    });
}

int tg_spmm(int64_t m, int64_t k, int64_t f, int64_t nnz, const int32_t* row_ptr,
            const int32_t* col_ind, const float* val, const float* b, int64_t ldb, float* c,
            int64_t ldc, tg_stream_t stream) {
    return tg_spmm_ex(m, k, f, nnz, row_ptr, col_ind, val, b, ldb, c, ldc, TG_PRECISION_EXACT,
                      stream);
}

}  // extern "C"
