// blocked.hip -- column-blocked CSR aggregation for graphs whose gathered
// feature matrix is larger than the L2 of an XCD.
//
// A plain CSR aggregation gathers B[col, :] for every nonzero; with 114.6M
// nonzeros over 233K source rows almost every gather misses L2 (4 MB per
// XCD) and the pass runs at HBM/MALL speed.  Cutting the columns into blocks
// of R source rows and running one pass per block keeps a pass's gathered
// lines (R x 128 bytes of the 32-column tile being processed) resident in
// L2, at the cost of re-reading and re-writing the output once per block.
// That trade pays when rows hold many entries per block (dense, high-degree
// graphs) and is skipped otherwise (resolve_block_rows).
//
// Layout in HBM: the nonzeros of block b, row i are
// bci/bv[brp[b*n + i] .. brp[b*n + i + 1]), blocks outermost, in the order
// they have in row i of the source structure.  brp[b*n + n] = brp[(b+1)*n],
// so block b's row pointer is the slice brp + b*n and ordinary row plans
// (absolute offsets) index it.  With blocks of at most 65,536 rows (every
// default) bci holds uint16 offsets within the entry's block, column -
// b * rows_per_block, and a pass reads B from the block's first row; wider
// blocks keep int32 columns.
#include "aggregate.hpp"
#include "common.hpp"
#include "spmm_plan.hpp"

#include <algorithm>

namespace tg {

namespace {

constexpr int kMaxBlocks = 64;   // one lane of a wave per column block
// Target rows per block, rounded down to equal blocks (n / ceil(n / target)).
// Measured at 233K nodes / 114.6M entries with tile-major gathers:
// * 32-column lane groups: 38912 rows x 128 bytes = 4.75 MB of one tile's
//   gathered lines; six equal blocks (38,828 rows) 11.13 / 10.06 / 15.18 ms
//   (GCN / SAGE / GAT); seven or eight equal blocks within 1%; blocks of
//   16,384 or 20,480 rows 4-12% slower.
// * 64-column lane groups read each block's indices once per two tiles (the
//   index stream, not the gathered bytes, bounds a pass) and gather two
//   lines per row, so they take smaller blocks: ten blocks of 23,297 rows
//   10.59 / 10.31 / 14.68 ms; eleven or twelve blocks within 1%; eight 6%
//   and six 16% slower.  Passes without a value stream (SAGE's mean, the
//   factored GCN) keep 32-column groups.
constexpr int64_t kDefaultBlockRows32 = 38912;
constexpr int64_t kDefaultBlockRows64 = 23552;

__device__ __forceinline__ int lanes_below(uint64_t m) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(
        static_cast<uint32_t>(m >> 32),
        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// c / d for 0 <= c < 2^31 and 0 < d < 2^31, d fixed per launch: through the
// double reciprocal (exact to one unit for these ranges) and one correction
// each way, in place of a 32-bit integer division sequence.
__device__ __forceinline__ int div_by(int c, int d, double inv_d) {
    int q = static_cast<int>(static_cast<double>(c) * inv_d);
    q -= (static_cast<int64_t>(q) * d > c) ? 1 : 0;
    q += (static_cast<int64_t>(q + 1) * d <= c) ? 1 : 0;
    return q;
}

// One wave per row.  The row is walked in 64-entry batches in order (groups
// of kSplitAhead batches are loaded at once, the next group's while the
// current one is placed: config-E reference-semantics GCN / SAGE forwards
// 11.3 ms with one batch ahead, 11.1 ms with groups of two or four).  The
// wave keeps one slot per block in LDS: COUNT, the block's entries so far
// (written to cnt[b*n + row] at the end); SCATTER, the block's next output
// position (starting at brp[b*n + row]).  A batch splits into runs of equal
// block (lane order); a run's entries take consecutive positions.
//   * COUNT: each run's last lane adds the run's length to its block's slot.
//     A row whose entries step back to an earlier block (the previous
//     entry's block comes from the lane below, or from the previous batch's
//     last lane) sets *disorder = 1.
//   * SCATTER, batch in block order (the common case: sorted rows): every
//     block has at most one run, so an entry's position is its block's slot
//     plus its rank in the run, and the run's last lane moves the slot past
//     the run.  Otherwise, per block b present in the batch, the entries of b
//     are ranked by the ballot bits below their lane (a stable partition).
constexpr int kSplitAhead = 4;
template <bool SCATTER>
__global__ __launch_bounds__(256) void block_split_kernel(
    const int32_t* __restrict__ rp, const int32_t* __restrict__ ci,
    const float* __restrict__ v, int64_t n, int rows_per_block, double inv_rows, int nb,
    int32_t* __restrict__ cnt_or_brp, int32_t* __restrict__ bci, uint16_t* __restrict__ bci16,
    float* __restrict__ bv, int32_t* __restrict__ disorder) {
    __shared__ int32_t slots[4][64];
    const int lane = threadIdx.x & 63;
    int32_t* slot = slots[threadIdx.x >> 6];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wave (no workgroup barrier below)
    const int s = rp[row], e = rp[row + 1];
    if (lane < nb) slot[lane] = SCATTER ? cnt_or_brp[static_cast<int64_t>(lane) * n + row] : 0;
    __builtin_amdgcn_wave_barrier();
    // the indices (and values) of kSplitAhead batches are loaded together,
    // the next group's behind the current group's placement
    int cq[kSplitAhead];
    float vq[kSplitAhead];
    auto load_group = [&](int i0, int (&c)[kSplitAhead], float (&vv)[kSplitAhead]) {
#pragma unroll
        for (int g = 0; g < kSplitAhead; ++g) {
            const int idx = i0 + g * 64 + lane;
            c[g] = idx < e ? ci[idx] : 0;
            vv[g] = 0.0f;
            if (SCATTER && bv) vv[g] = idx < e ? v[idx] : 0.0f;
        }
    };
    load_group(s, cq, vq);
    int prev_last = -1;  // the block of the previous batch's last entry
    bool back_seen = false;
    for (int i0 = s; i0 < e; i0 += 64 * kSplitAhead) {
        int cn[kSplitAhead];
        float vn[kSplitAhead];
        const bool more = i0 + 64 * kSplitAhead < e;  // uniform
        if (more) load_group(i0 + 64 * kSplitAhead, cn, vn);
#pragma unroll
        for (int g = 0; g < kSplitAhead; ++g) {
            const int i = i0 + g * 64;
            if (i >= e) break;  // uniform
            const int idx = i + lane;
            const bool valid = idx < e;
            const int c = cq[g];
            const float val = vq[g];
            const int blk = valid ? div_by(c, rows_per_block, inv_rows) : -1;
            const int below = __shfl_up(blk, 1);
            const int above = __shfl_down(blk, 1);
            const int pb = lane == 0 ? prev_last : below;
            const bool in_order = __ballot(valid && pb > blk) == 0;
            prev_last = __shfl(blk, 63);  // a full batch continues; the last one ends the row
            // runs: a start where the block changes from the lane below, an
            // end where it changes to the lane above (invalid lanes hold -1)
            const uint64_t starts = __ballot(valid && (lane == 0 || below != blk));
            const bool run_end = valid && (lane == 63 || above != blk);
            const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
            const int rank = lane - (63 - __clzll(starts & upto));  // valid lanes only
            if (!SCATTER) {
                back_seen |= !in_order;
                if (run_end) atomicAdd(&slot[blk], rank + 1);
                continue;
            }
            int pos = 0;
            if (in_order) {
                if (valid) pos = slot[blk] + rank;
                __builtin_amdgcn_wave_barrier();
                if (run_end) slot[blk] = pos + 1;
            } else {
                for (int b = 0; b < nb; ++b) {
                    const uint64_t m = __ballot(blk == b);
                    if (m == 0) continue;  // uniform: the ballot is the wave's
                    const int base = slot[b];
                    __builtin_amdgcn_wave_barrier();
                    if (blk == b) pos = base + lanes_below(m);
                    if (lane == b) slot[b] = base + __popcll(m);
                    __builtin_amdgcn_wave_barrier();
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (valid) {
                if (bci16)
                    bci16[pos] = static_cast<uint16_t>(c - blk * rows_per_block);
                else
                    bci[pos] = c;
                if (bv) bv[pos] = val;
            }
        }
        if (more) {
#pragma unroll
            for (int g = 0; g < kSplitAhead; ++g) {
                cq[g] = cn[g];
                vq[g] = vn[g];
            }
        }
    }
    if (!SCATTER) {
        if (back_seen && lane == 0) atomicOr(disorder, 1);
        __builtin_amdgcn_wave_barrier();
        if (lane < nb) cnt_or_brp[static_cast<int64_t>(lane) * n + row] = slot[lane];
    }
}

// ---------------------------------------------------------------------------
// Sorted-row split.  When every row's columns are non-decreasing (every CSR
// edge_list_to_csr builds), a block's entries in a row form one contiguous
// run, so the split reduces to the runs' starts: entry j starts the runs of
// blocks (block(c[j-1]), block(c[j])], with block(c[-1]) = -1; blocks past
// the last entry's start at the row's end.  G lanes share a row (16, 64 or a
// 256-thread workgroup by row length), lane l taking entries l, l + G, ...
// with kSortedU of them loaded per step and the next step's loaded ahead;
// the starts collect in LDS.  The count pass writes each block's count and
// start, the scatter pass copies every entry to its block's row segment at
// its rank in the run.  Its purpose is vdiag: every row i also holds a
// virtual entry (column i, no value) at its sorted position, before its
// first column > i, which gives A + I's blocked copy straight from A (the
// general kernel above handles any order, without that entry).  A row found
// out of order sets flags[0], one with a diagonal flags[1]; it then counts
// its whole length in block 0 (the totals stay those of a valid split), the
// scatter pass writes nothing and the caller takes another path.
// ---------------------------------------------------------------------------
constexpr int kShortSplit = 512;
constexpr int kLongSplit = 4096;

struct SortedSplit {
    const int32_t* rp;
    const int32_t* ci;
    const float* v;           // scatter: values to copy, or null
    int64_t n;
    int rows_per_block;
    double inv_rows;
    int nb;
    int vdiag;
    const int32_t* long_list;  // rows longer than kLongSplit, *long_count of them
    const int32_t* long_count;
    int32_t* cnt;              // count pass: [nb * n] entries per block and row
    const int32_t* brp;        // scatter pass: the scanned counts
    int32_t* starts;           // [nb * n] each block's first position in the row
    int32_t* ins;              // [n] (vdiag) the virtual entry's position in the row
    int32_t* bci;
    uint16_t* bci16;
    float* bv;
    int32_t* flags;            // [0] a row out of order, [1] (vdiag) a row with a diagonal
};

template <int G>
__device__ __forceinline__ void group_sync() {
    if constexpr (G == 256)
        __syncthreads();
    else
        __builtin_amdgcn_wave_barrier();  // the group's lanes are in one wave
}

__device__ __forceinline__ int block_of(int c, const SortedSplit& a) {
    const int b = div_by(c < 0 ? 0 : c, a.rows_per_block, a.inv_rows);
    return b < a.nb ? b : a.nb - 1;  // in bounds whatever the column
}

// Entries of one step: lane l of the group takes entries j0 + u*G + l,
// u < kSortedU (coalesced across the group), the next step's loaded before
// the current one is placed.
constexpr int kSortedU = 8;

struct SortedStep {
    int c[kSortedU];
    int pc[kSortedU];  // the previous entries, loaded where no shuffle reaches them
    float x[kSortedU];
};

// W: the shuffle width (the group, or one wave of a workgroup-wide group);
// the first lane of each W-lane span loads its entries' predecessors.
template <int G, bool VALUES, bool PREV>
__device__ __forceinline__ void load_step(const SortedSplit& a, int s, int len, int j0, int lane,
                                          SortedStep& t) {
    constexpr int W = G < 64 ? G : 64;
#pragma unroll
    for (int u = 0; u < kSortedU; ++u) {
        const int j = j0 + u * G + lane;
        t.c[u] = j < len ? a.ci[s + j] : 0;
        if (VALUES) t.x[u] = j < len ? a.v[s + j] : 0.0f;
        if (PREV) t.pc[u] = (lane % W == 0 && j > 0 && j <= len) ? a.ci[s + j - 1] : -1;
    }
}

template <int G, bool SCATTER>
__device__ __forceinline__ void split_sorted_row(const SortedSplit& a, int64_t row, int lane,
                                                 int32_t* slot, int32_t* misc) {
    constexpr int W = G < 64 ? G : 64;
    constexpr int STEP = G * kSortedU;
    const int64_t n = a.n;
    const int nb = a.nb;
    const int s = a.rp[row], e = a.rp[row + 1], len = e - s;
    const int i = static_cast<int>(row);
    if constexpr (!SCATTER) {
        for (int b = lane; b < nb; b += G) slot[b] = len;
        if (lane == 0) {
            misc[0] = len;  // the virtual entry's position: before the first column > i
            misc[1] = 0;
        }
        group_sync<G>();
        int bad = 0;
        SortedStep cur, nxt;
        load_step<G, false, true>(a, s, len, 0, lane, cur);
        for (int j0 = 0; j0 < len; j0 += STEP) {
            if (j0 + STEP < len) load_step<G, false, true>(a, s, len, j0 + STEP, lane, nxt);
#pragma unroll
            for (int u = 0; u < kSortedU; ++u) {
                const int j = j0 + u * G + lane;
                // the previous entry: the lane below's, or the loaded one
                const int up = __shfl_up(cur.c[u], 1, W);
                const int pc = lane % W != 0 ? up : cur.pc[u];
                if (j < len) {
                    const int c = cur.c[u];
                    const int cb = block_of(c, a);
                    const int pb = j > 0 ? block_of(pc, a) : -1;
                    bad |= (j > 0 && pc > c) ? 1 : 0;
                    if (a.vdiag) {
                        bad |= c == i ? 2 : 0;
                        if ((j == 0 || pc < i) && c > i) misc[0] = j;
                    }
                    for (int b = pb + 1; b <= cb; ++b) slot[b] = j;
                }
            }
            cur = nxt;
        }
        if (bad) atomicOr(&misc[1], bad);
        group_sync<G>();
        const int flag = misc[1];
        const int d = a.vdiag ? block_of(i, a) : nb;  // the virtual entry's block
        if (lane == 0 && (flag & 1)) atomicOr(&a.flags[0], 1);
        if (lane == 0 && (flag & 2)) atomicOr(&a.flags[1], 1);
        for (int b = lane; b < nb; b += G) {
            const int st = slot[b] + (b > d ? 1 : 0);
            const int nx = (b + 1 < nb ? slot[b + 1] : len) + (b + 1 > d ? 1 : 0);
            const int64_t o = static_cast<int64_t>(b) * n + row;
            a.cnt[o] = flag ? (b == 0 ? len + a.vdiag : 0) : nx - st;
            a.starts[o] = flag ? 0 : st;
        }
        if (a.vdiag && lane == 0) a.ins[row] = misc[0];
        group_sync<G>();  // the slots are reused by the group's next row
    } else {
        // out position of the entry at (virtual) row position jv in block b:
        // brp[b*n + row] + jv - starts[b*n + row]
        for (int b = lane; b < nb; b += G) {
            const int64_t o = static_cast<int64_t>(b) * n + row;
            slot[b] = a.brp[o] - a.starts[o];
        }
        group_sync<G>();
        const int R = a.rows_per_block;
        SortedStep cur, nxt;
        const bool vals = a.bv != nullptr;
        if (vals)
            load_step<G, true, false>(a, s, len, 0, lane, cur);
        else
            load_step<G, false, false>(a, s, len, 0, lane, cur);
        for (int j0 = 0; j0 < len; j0 += STEP) {
            if (j0 + STEP < len) {
                if (vals)
                    load_step<G, true, false>(a, s, len, j0 + STEP, lane, nxt);
                else
                    load_step<G, false, false>(a, s, len, j0 + STEP, lane, nxt);
            }
#pragma unroll
            for (int u = 0; u < kSortedU; ++u) {
                const int j = j0 + u * G + lane;
                if (j >= len) continue;
                const int c = cur.c[u];
                const int cb = block_of(c, a);
                const int out = slot[cb] + j + (a.vdiag && c > i ? 1 : 0);
                if (a.bci16)
                    a.bci16[out] = static_cast<uint16_t>(c - cb * R);
                else
                    a.bci[out] = c;
                if (vals) a.bv[out] = cur.x[u];
            }
            cur = nxt;
        }
        if (a.vdiag && lane == 0) {
            const int d = block_of(i, a);
            const int out = slot[d] + a.ins[row];
            if (a.bci16)
                a.bci16[out] = static_cast<uint16_t>(i - d * R);
            else
                a.bci[out] = i;
        }
        group_sync<G>();
    }
}

// Rows by length class: G = 16 lanes for rows of at most kShortSplit
// entries, a wave (G = 64) up to kLongSplit, so no row takes more than eight
// steps of its group (config-E count + scatter: 0.75 ms with 16-lane groups
// and 4 entries per lane up to kLongSplit, 0.65 ms so); longer rows:
// split_sorted_long_kernel.
template <int G, bool SCATTER>
__global__ __launch_bounds__(256) void split_sorted_kernel(SortedSplit a) {
    constexpr int NG = 256 / G;
    __shared__ int32_t slots[NG][kMaxBlocks];
    __shared__ int32_t misc[NG][2];
    if (SCATTER && (a.flags[0] | a.flags[1])) return;  // the general split runs instead
    const int grp = threadIdx.x / G;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * NG + grp;
    if (row >= a.n) return;
    const int len = a.rp[row + 1] - a.rp[row];
    if (G == 16 ? len > kShortSplit : (len <= kShortSplit || len > kLongSplit)) return;
    split_sorted_row<G, SCATTER>(a, row, threadIdx.x % G, slots[grp], misc[grp]);
}

// The listed longer rows: one workgroup each, grid-stride over the list.
template <bool SCATTER>
__global__ __launch_bounds__(256) void split_sorted_long_kernel(SortedSplit a) {
    __shared__ int32_t slot[kMaxBlocks];
    __shared__ int32_t misc[2];
    if (SCATTER && (a.flags[0] | a.flags[1])) return;
    const int64_t count = *a.long_count;
    for (int64_t t = blockIdx.x; t < count; t += gridDim.x)
        split_sorted_row<256, SCATTER>(a, a.long_list[t], static_cast<int>(threadIdx.x), slot,
                                       misc);
}

__global__ __launch_bounds__(256) void split_long_rows_kernel(const int32_t* __restrict__ rp,
                                                              int64_t n,
                                                              int32_t* __restrict__ list,
                                                              int32_t* __restrict__ count) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < n && rp[r + 1] - rp[r] > kLongSplit) list[atomicAdd(count, 1)] = static_cast<int32_t>(r);
}

}  // namespace

int64_t resolve_block_rows(int64_t requested, int64_t n, int64_t nnz, int group_cols) {
    if (requested == 0 || n <= 0) return 0;
    const int64_t target = group_cols == 64 ? kDefaultBlockRows64 : kDefaultBlockRows32;
    int64_t r = requested > 0 ? requested : ceil_div(n, ceil_div(n, target));
    r = std::max<int64_t>(r, ceil_div(n, kMaxBlocks));
    const int64_t nb = ceil_div(n, r);
    if (nb < 2) return 0;
    if (requested < 0 && nnz < 8 * n * nb) return 0;
    return r;
}

namespace {

// The split's temporaries: counts, the scan's temp, flags ([0] a row out of
// order, [1] a diagonal (vdiag), [2] the general split's disorder, [3] the
// long-row count), the sorted split's starts, virtual positions and
// long-row list.
struct SplitTemps {
    int32_t *cnt, *flags, *starts, *ins, *long_list;
    int64_t* scan_tmp;
};

SplitTemps carve_split(Carver& c, int64_t n, int64_t nb) {
    SplitTemps t;
    t.cnt = c.take<int32_t>(nb * n);
    t.scan_tmp = c.take<int64_t>(scan_temp_elems(nb * n));
    t.flags = c.take<int32_t>(4);
    t.starts = c.take<int32_t>(nb * n);
    t.ins = c.take<int32_t>(n);
    t.long_list = c.take<int32_t>(n);
    return t;
}

// Shapes the blocked copy for n rows and nnz entries and returns its
// temporaries.
SplitTemps setup_blocked(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                         bool weighted, int64_t rows_per_block) {
    require(n > 0 && rows_per_block > 0, "blocked CSR: empty structure or block");
    require(nnz >= 0 && nnz < (int64_t(1) << 31), "blocked CSR: nnz must be < 2^31");
    const int64_t nb = ceil_div(n, rows_per_block);
    require(nb <= kMaxBlocks, "blocked CSR: at most 64 column blocks");
    require(nb * n < (int64_t(1) << 31), "blocked CSR: blocks x rows must be < 2^31");
    require(rp != nullptr, "blocked CSR: null structure");
    bk.n = n;
    bk.nnz = nnz;
    bk.rows_per_block = rows_per_block;
    bk.n_blocks = nb;
    bk.rp = rp;
    bk.weighted = weighted;
    bk.brp.reserve(static_cast<size_t>(nb * n + 1) * sizeof(int32_t));
    bk.idx16 = rows_per_block <= 65536;
    bk.bci.reserve(static_cast<size_t>(std::max<int64_t>(nnz, 1)) *
                   (bk.idx16 ? sizeof(uint16_t) : sizeof(int32_t)));
    if (weighted) bk.bv.reserve(static_cast<size_t>(std::max<int64_t>(nnz, 1)) * sizeof(float));
    Carver cv(nullptr, 0);
    carve_split(cv, n, nb);
    bk.scratch.reserve(cv.bytes());
    Carver c(bk.scratch.get(), bk.scratch.size());
    // host results: the plans' totals (4 per block), then the flags
    bk.host.reserve(static_cast<size_t>(4 * nb + 2) * sizeof(int64_t));
    bk.plans.resize(static_cast<size_t>(nb));
    for (auto& p : bk.plans)
        if (!p) p = std::make_unique<tg_spmm_plan_s>();
    return carve_split(c, n, nb);
}

// One plan per block, all built by one launch per step and one
// synchronisation, which also brings back the flags enqueued before it
// (config-E reference-semantics forwards: per-block builds, about ten
// launches each, cost 0.25-0.4 ms more).
void build_block_plans(BlockedCSR& bk, int64_t max_f, int64_t chunk, hipStream_t s) {
    std::vector<tg_spmm_plan_s*> plans(bk.plans.size());
    for (size_t b = 0; b < plans.size(); ++b) plans[b] = bk.plans[b].get();
    build_plans_multi(plans.data(), static_cast<int>(bk.n_blocks), bk.n, bk.nnz,
                      bk.brp.as<int32_t>(), max_f, chunk, bk.plan_scratch,
                      bk.host.as<int64_t>(), s);
}

// The sorted-row split (with or without the virtual diagonal); false when
// some row is out of order or, with vdiag, has a diagonal (the copy is then
// incomplete and the caller takes another path).
bool split_sorted(BlockedCSR& bk, const SplitTemps& t, const int32_t* rp, const int32_t* ci,
                  const float* v, int64_t nnz_src, bool vdiag, int64_t max_f, int64_t chunk,
                  hipStream_t s) {
    const int64_t n = bk.n, nb = bk.n_blocks;
    fill_i32(t.flags, 4, 0, s);
    split_long_rows_kernel<<<static_cast<unsigned>(ceil_div(n, 256)), 256, 0, s>>>(
        rp, n, t.long_list, t.flags + 3);
    TG_LAUNCH_CHECK();
    SortedSplit a{};
    a.rp = rp;
    a.ci = ci;
    a.v = v;
    a.n = n;
    a.rows_per_block = static_cast<int>(bk.rows_per_block);
    a.inv_rows = 1.0 / static_cast<double>(bk.rows_per_block);
    a.nb = static_cast<int>(nb);
    a.vdiag = vdiag ? 1 : 0;
    a.long_list = t.long_list;
    a.long_count = t.flags + 3;
    a.cnt = t.cnt;
    a.starts = t.starts;
    a.ins = t.ins;
    a.flags = t.flags;
    // grid-stride over at most nnz / (kLongSplit + 1) long rows
    const unsigned long_grid =
        static_cast<unsigned>(std::min<int64_t>(nnz_src / (kLongSplit + 1) + 1, 1024));
    const unsigned grid16 = static_cast<unsigned>(ceil_div(n, 16));
    const unsigned grid64 = static_cast<unsigned>(ceil_div(n, 4));
    split_sorted_kernel<16, false><<<grid16, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    split_sorted_kernel<64, false><<<grid64, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    split_sorted_long_kernel<false><<<long_grid, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    int32_t* brp = bk.brp.as<int32_t>();
    exclusive_scan_i32(t.cnt, brp, nb * n, t.scan_tmp, s);
    a.brp = brp;
    a.bci = bk.idx16 ? nullptr : bk.bci.as<int32_t>();
    a.bci16 = bk.idx16 ? bk.bci.as<uint16_t>() : nullptr;
    a.bv = v ? bk.bv.as<float>() : nullptr;
    split_sorted_kernel<16, true><<<grid16, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    split_sorted_kernel<64, true><<<grid64, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    split_sorted_long_kernel<true><<<long_grid, 256, 0, s>>>(a);
    TG_LAUNCH_CHECK();
    int32_t* hf = reinterpret_cast<int32_t*>(bk.host.as<int64_t>() + 4 * nb);
    TG_HIP(hipMemcpyAsync(hf, t.flags, 2 * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    build_block_plans(bk, max_f, chunk, s);
    return hf[0] == 0 && hf[1] == 0;
}

// The general split (any order), with the disorder flag: count, scan,
// scatter, plans.
void split_general(BlockedCSR& bk, const SplitTemps& t, const int32_t* rp, const int32_t* ci,
                   const float* v, int64_t max_f, int64_t chunk, hipStream_t s) {
    const int64_t n = bk.n, nb = bk.n_blocks;
    const int R = static_cast<int>(bk.rows_per_block);
    int32_t* disorder = t.flags + 2;
    fill_i32(disorder, 1, 0, s);
    const unsigned grid = static_cast<unsigned>(ceil_div(n, 4));
    const double inv_rows = 1.0 / static_cast<double>(R);
    block_split_kernel<false><<<grid, 256, 0, s>>>(rp, ci, v, n, R, inv_rows,
                                                   static_cast<int>(nb), t.cnt, nullptr, nullptr,
                                                   nullptr, disorder);
    TG_LAUNCH_CHECK();
    int32_t* brp = bk.brp.as<int32_t>();
    exclusive_scan_i32(t.cnt, brp, nb * n, t.scan_tmp, s);
    block_split_kernel<true><<<grid, 256, 0, s>>>(rp, ci, v, n, R, inv_rows,
                                                  static_cast<int>(nb), brp,
                                                  bk.idx16 ? nullptr : bk.bci.as<int32_t>(),
                                                  bk.idx16 ? bk.bci.as<uint16_t>() : nullptr,
                                                  v ? bk.bv.as<float>() : nullptr, nullptr);
    TG_LAUNCH_CHECK();
    int32_t* hf = reinterpret_cast<int32_t*>(bk.host.as<int64_t>() + 4 * nb);
    TG_HIP(hipMemcpyAsync(hf, disorder, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    build_block_plans(bk, max_f, chunk, s);
    bk.in_order = hf[0] == 0;
}

}  // namespace

void build_blocked(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                   const int32_t* ci, const float* v, int64_t rows_per_block, int64_t max_f,
                   hipStream_t s, int64_t chunk) {
    const SplitTemps t = setup_blocked(bk, n, nnz, rp, v != nullptr, rows_per_block);
    require(nnz == 0 || ci != nullptr, "blocked CSR: null structure");
    // (the sorted-row split is no faster here: config-E count + scatter
    // 0.65 ms against 0.63 ms; it serves the virtual diagonal below)
    split_general(bk, t, rp, ci, v, max_f, chunk, s);
}

bool build_blocked_self_loops(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                              const int32_t* ci, int64_t rows_per_block, int64_t max_f,
                              hipStream_t s, int64_t chunk) {
    require(nnz + n < (int64_t(1) << 31), "blocked CSR: nnz + n must be < 2^31");
    const SplitTemps t = setup_blocked(bk, n, nnz + n, rp, false, rows_per_block);
    require(nnz == 0 || ci != nullptr, "blocked CSR: null structure");
    if (!split_sorted(bk, t, rp, ci, nullptr, nnz, true, max_f, chunk, s)) return false;
    bk.in_order = true;
    return true;
}

void run_aggregate_blocked(const BlockedCSR& bk, int64_t f, const float* b, int64_t ldb,
                           float* c, int64_t ldc, const AggEpilogue& epi, hipStream_t s) {
    require(!epi.max, "blocked aggregation: max is not supported");
    require(!epi.acc && !epi.skip_empty, "blocked aggregation: pass flags are set per block");
    if (bk.n == 0 || f == 0) return;
    const int32_t* bci = bk.idx16 ? nullptr : bk.bci.as<int32_t>();
    // attention passes compute their weights (no value stream)
    const float* bv = epi.att_dst == nullptr && bk.weighted ? bk.bv.as<float>() : nullptr;
    // One launch per block over all column groups of f (grid.y), blocks in
    // order: the first pass stores every row (zero where the block has no
    // entries), middle passes touch only rows with entries, the last pass
    // adds and applies the epilogue to every row.  64-column groups only
    // where a group has two tiles' worth of columns and, for attention
    // passes, lies in one head.
    const bool per_head = epi.att_dst != nullptr;
    const bool wide = bk.group_cols == 64 && f > 32 &&
                      (!per_head || epi.w_head_cols >= f || epi.w_head_cols % 64 == 0);
    const int group_cols = wide ? 64 : 32;
    for (int64_t blk = 0; blk < bk.n_blocks; ++blk) {
        const bool first = blk == 0, last = blk + 1 == bk.n_blocks;
        AggEpilogue e;
        if (last) {
            e = epi;
            if (e.mean) e.deg_rp = bk.rp;
        }
        e.acc = first ? 0 : 1;
        e.skip_empty = (!first && !last) ? 1 : 0;
        // the operands' layouts, in every pass
        e.b_tile_stride = epi.b_tile_stride;
        e.w_head_cols = epi.w_head_cols;
        e.exact_exp = epi.exact_exp;
        e.att_src = epi.att_src;
        e.att_dst = epi.att_dst;
        e.att_max = epi.att_max;
        e.att_rinv = epi.att_rinv;
        e.att_heads = epi.att_heads;
        e.att_slope = epi.att_slope;
        // 16-bit indices count from the block's first source row
        const int64_t r0 = bk.idx16 ? blk * bk.rows_per_block : 0;
        const float* bb = b + r0 * (epi.b_tile_stride > 0 ? 32 : ldb);
        if (bk.idx16) {
            e.ci16 = bk.bci.as<uint16_t>();
            if (e.att_dst) e.att_dst = epi.att_dst + r0 * epi.att_heads;
        }
        run_aggregate(*bk.plans[blk], f, bci, bv, bb, ldb, c, ldc, e, s, group_cols);
    }
}

}  // namespace tg
