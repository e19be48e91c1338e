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
// Flat split, for rows whose entries are in block order (sorted rows: every
// CSR edge_list_to_csr builds).  A block's entries in a row are then one
// run, and the split reduces to each run's start: entry k starts the runs of
// blocks (block(c[k-1]), block(c[k])] of its row (all blocks up to block(c[k])
// when k starts the row).  Instead of a group of lanes per row (bound by the
// row-level latency of dependent loads: config E's count + scatter 0.63 ms
// with the general kernel, a read-only pass one wave per row 0.13 ms), both
// passes stream col_ind one entry per thread, coalesced, and find an
// entry's row from a bitmap of row starts: with rank = the number of row
// starts at or before k (a scan over 64-entry slices plus a popcount within
// the slice), the row is the rank-th non-empty row.  The count pass writes
// the run starts (every start preset to the row's length, for the blocks
// past its last entry); counts, their scan and the output bases follow per
// (block, row); the scatter pass writes every entry at its base plus its
// position.  An entry that steps back to an earlier block sets flags[0] (the
// caller then runs the general split).  With vdiag every row i also holds a
// virtual entry (column i, no value) before its first column > i: the
// diagonal of A + I for an A without one; a diagonal in A sets flags[1], a
// row out of order anywhere flags[0].
// ---------------------------------------------------------------------------
struct FlatSplit {
    const int32_t* rp;
    const int32_t* ci;
    const float* v;             // scatter: values to copy, or null
    int64_t n, nnz;
    int rows_per_block;
    double inv_rows;
    int nb;
    int vdiag;
    const uint64_t* bits;       // bit k: entry k starts a (non-empty) row
    const int32_t* slice_rank;  // row starts before each 64-entry slice
    const int32_t* nz_rows;     // the non-empty rows in order
    int32_t* starts;            // [nb * n] each block's first position in the row
    int32_t* ins;               // [n] (vdiag) the virtual entry's position
    const int32_t* obase;       // scatter: [nb * n] brp - starts - rp[row]
    int32_t* bci;
    uint16_t* bci16;
    float* bv;
    int32_t* flags;             // [0] an entry out of block order, [1] (vdiag) a diagonal,
                                // [3] (row split) rows longer than kRowCap
    int32_t* long_rows;         // row split: those rows
};

__device__ __forceinline__ int block_of(int c, const FlatSplit& a) {
    const int b = div_by(c < 0 ? 0 : c, a.rows_per_block, a.inv_rows);
    return b < a.nb ? b : a.nb - 1;  // in bounds whatever the column
}

// Bit rp[r] for every non-empty row r, the non-empty flags; the row's
// length as every block's start (blocks past its last entry), and as the
// virtual entry's position (a row whose columns are all < i).
__global__ __launch_bounds__(256) void flat_marks_kernel(FlatSplit a, uint32_t* __restrict__ bits32,
                                                         int32_t* __restrict__ nonempty) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= a.n) return;
    const int s = a.rp[r], e = a.rp[r + 1];
    nonempty[r] = e > s ? 1 : 0;
    if (e > s && s >= 0 && s < a.nnz) atomicOr(&bits32[s >> 5], 1u << (s & 31));
    for (int b = 0; b < a.nb; ++b) a.starts[static_cast<int64_t>(b) * a.n + r] = e - s;
    if (a.vdiag) a.ins[r] = e - s;
}

__global__ __launch_bounds__(256) void flat_nzrows_kernel(const int32_t* __restrict__ rp, int64_t n,
                                                          const int32_t* __restrict__ nzrank,
                                                          int32_t* __restrict__ nz_rows) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < n && rp[r + 1] > rp[r]) nz_rows[nzrank[r]] = static_cast<int32_t>(r);
}

__global__ __launch_bounds__(256) void flat_popc_kernel(const uint64_t* __restrict__ bits,
                                                        int64_t slices, int32_t* __restrict__ popc) {
    const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (w < slices) popc[w] = __popcll(bits[w]);
}

// Each wave takes kFlatSU consecutive 64-entry slices (lane l: entry l of
// each), with every slice's loads issued before the dependent ones: an
// entry's row is a chain of loads (bitmap and slice rank, then the
// non-empty row, then its row pointer), and one slice per wave left that
// chain's latency exposed (config-E count and scatter passes 0.45 ms each).
constexpr int kFlatSU = 8;

struct FlatRows {
    int c[kFlatSU];     // the entries' columns
    int row[kFlatSU];   // their rows (valid entries)
    int pos[kFlatSU];   // their positions in the row
    bool first[kFlatSU];  // an entry that starts its row
    bool valid[kFlatSU];
};

// The wave's slices w0 .. w0 + kFlatSU - 1 (w0 < slices): columns, rows and
// positions; an entry whose rank finds no row sets flags[0].
__device__ __forceinline__ void flat_rows(const FlatSplit& a, int64_t w0, int lane, FlatRows& f) {
    const int64_t slices = (a.nnz + 63) >> 6;
    const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
    uint64_t word[kFlatSU];
    int srank[kFlatSU];
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        const int64_t w = w0 + u;
        const int64_t k = w * 64 + lane;
        f.valid[u] = k < a.nnz;
        f.c[u] = f.valid[u] ? a.ci[k] : 0;
        word[u] = w < slices ? a.bits[w] : 0ull;
        srank[u] = w < slices ? a.slice_rank[w] : 0;
    }
    int rank[kFlatSU];
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        rank[u] = srank[u] + __popcll(word[u] & upto);
        f.first[u] = (word[u] >> lane) & 1;
        if (f.valid[u] && rank[u] < 1) {
            atomicOr(&a.flags[0], 1);
            f.valid[u] = false;
        }
    }
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) f.row[u] = f.valid[u] ? a.nz_rows[rank[u] - 1] : 0;
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u)
        f.pos[u] = static_cast<int>((w0 + u) * 64 + lane - a.rp[f.row[u]]);
}

__global__ __launch_bounds__(256) void flat_count_kernel(FlatSplit a) {
    const int lane = threadIdx.x & 63;
    const int64_t w0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kFlatSU;
    if (w0 * 64 >= a.nnz) return;  // uniform per wave
    FlatRows f;
    flat_rows(a, w0, lane, f);
    // each entry's predecessor: the lane below, or the previous slice's last
    // lane, or (the wave's first entry) a load
    const int pc0 = (lane == 0 && w0 > 0) ? a.ci[w0 * 64 - 1] : 0;
    int blk[kFlatSU], last[kFlatSU], lastb[kFlatSU];
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        blk[u] = block_of(f.c[u], a);
        last[u] = __shfl(f.c[u], 63, 64);
        lastb[u] = __shfl(blk[u], 63, 64);
    }
    const int pb0 = block_of(pc0, a);
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        int pc = __shfl_up(f.c[u], 1, 64);
        int pbk = __shfl_up(blk[u], 1, 64);
        if (lane == 0) {
            pc = u == 0 ? pc0 : last[u > 0 ? u - 1 : 0];
            pbk = u == 0 ? pb0 : lastb[u > 0 ? u - 1 : 0];
        }
        if (!f.valid[u]) continue;
        const int c = f.c[u], row = f.row[u], pos = f.pos[u];
        const int b = blk[u];
        const int pb = f.first[u] ? -1 : pbk;
        if (pb > b) atomicOr(&a.flags[0], 1);
        for (int x = pb + 1; x <= b; ++x) a.starts[static_cast<int64_t>(x) * a.n + row] = pos;
        if (a.vdiag) {
            if (c == row) atomicOr(&a.flags[1], 1);
            // the virtual entry goes before the row's first column > i: one
            // such position only in a sorted row (out of order within a
            // block, decline as for block order)
            if (!f.first[u] && pc > c) atomicOr(&a.flags[0], 1);
            if ((f.first[u] || pc < row) && c > row) a.ins[row] = pos;
        }
    }
}

// Per (block, row): the count (the virtual entry in its block), or, after
// a flagged count pass, the row's whole length in block 0.
__global__ __launch_bounds__(256) void flat_counts_kernel(FlatSplit a, int32_t* __restrict__ cnt) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= a.n * a.nb) return;
    const int b = static_cast<int>(t / a.n);
    const int64_t r = t - static_cast<int64_t>(b) * a.n;
    const int len = a.rp[r + 1] - a.rp[r];
    if (a.flags[0] | a.flags[1]) {
        cnt[t] = b == 0 ? len + a.vdiag : 0;
        return;
    }
    const int st = a.starts[t];
    const int nx = b + 1 < a.nb ? a.starts[t + a.n] : len;
    const int d = a.vdiag ? block_of(static_cast<int>(r), a) : -1;
    cnt[t] = nx - st + (b == d ? 1 : 0);
}

// obase = brp - start - rp[row] (in place of the counts, which the scan has
// consumed): entry k of the block's run goes to obase + k (+1 past the
// virtual entry in its block).
__global__ __launch_bounds__(256) void flat_bases_kernel(FlatSplit a, const int32_t* __restrict__ brp,
                                                         int32_t* __restrict__ obase) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= a.n * a.nb) return;
    const int b = static_cast<int>(t / a.n);
    const int64_t r = t - static_cast<int64_t>(b) * a.n;
    obase[t] = brp[t] - a.starts[t] - a.rp[r];
}

__global__ __launch_bounds__(256) void flat_scatter_kernel(FlatSplit a) {
    if (a.flags[0] | a.flags[1]) return;  // the caller runs another split
    const int lane = threadIdx.x & 63;
    const int64_t w0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kFlatSU;
    if (w0 * 64 >= a.nnz) return;
    FlatRows f;
    flat_rows(a, w0, lane, f);
    float x[kFlatSU];
    int out[kFlatSU], b[kFlatSU];
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        const int64_t k = (w0 + u) * 64 + lane;
        x[u] = (a.bv && f.valid[u]) ? a.v[k] : 0.0f;
        b[u] = block_of(f.c[u], a);
        out[u] = f.valid[u] ? a.obase[static_cast<int64_t>(b[u]) * a.n + f.row[u]] : 0;
    }
#pragma unroll
    for (int u = 0; u < kFlatSU; ++u) {
        if (!f.valid[u]) continue;
        const int c = f.c[u], row = f.row[u];
        int o = out[u] + static_cast<int>((w0 + u) * 64 + lane);
        if (a.vdiag && c > row && b[u] == block_of(row, a)) ++o;
        if (a.bci16)
            a.bci16[o] = static_cast<uint16_t>(c - b[u] * a.rows_per_block);
        else
            a.bci[o] = c;
        if (a.bv) a.bv[o] = x[u];
    }
}

// vdiag: each row's virtual entry.
__global__ __launch_bounds__(256) void flat_diag_kernel(FlatSplit a, const int32_t* __restrict__ brp) {
    if (a.flags[0] | a.flags[1]) return;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= a.n) return;
    const int i = static_cast<int>(r);
    const int d = block_of(i, a);
    const int64_t t = static_cast<int64_t>(d) * a.n + r;
    const int out = brp[t] + a.ins[r] - a.starts[t];
    if (a.bci16)
        a.bci16[out] = static_cast<uint16_t>(i - d * a.rows_per_block);
    else
        a.bci[out] = i;
}

// ---------------------------------------------------------------------------
// Row split, for long sorted rows (at least kRowSplitMinAvg entries per row
// on average).  A group of lanes per row finds every block's start in the
// row by binary search over its sorted columns (a running maximum keeps the
// starts non-decreasing, so a row's counts sum to its length whatever its
// order); the counts' scan gives the copy's offsets, and one wavefront per
// row streams the row's entries to them, each entry's block start and base
// from the lane that loaded them.  No pass reads every entry to count it:
// the flat split reads each column twice (count and scatter) and finds its
// row through a chain of dependent loads (config E's A + I: flat count 0.22
// + scatter 0.25 ms, plus the flat split's bitmap, rank and non-empty-row
// passes).  The scatter checks the order as it goes: a column below its
// predecessor sets flags[0]; with vdiag a diagonal sets flags[1].
// ---------------------------------------------------------------------------
constexpr int64_t kRowSplitMinAvg = 64;
// entries of a row that its own wavefront writes; the rest of a longer row
// is shared by the four wavefronts of one of the scatter's first kLongWgs
// workgroups
constexpr int kRowCap = 2048;
constexpr int kLongWgs = 1024;

// The first position in ci[lo, hi) whose column is >= key (ci[lo, hi)
// sorted), by 9-ary search: each round loads 8 evenly spaced columns of the
// range at once and keeps the ninth between the last one below the key and
// the first one at or above it, until at most 8 are left, which are loaded
// and counted.  Three dependent rounds of loads for a 492-entry row, five for
// 20,000 entries, against 9 and 15 probes of a binary search (config E's
// row search 0.12 ms with those).  Whatever the order the result stays in
// [lo, hi] and every load inside the range.
__device__ __forceinline__ int lower_bound_col(const int32_t* __restrict__ ci, int lo, int hi,
                                               int64_t key) {
    int a = lo, b = hi;  // the answer is in [a, b]
    while (b - a > 8) {
        // positions a + floor((i + 1) w / 9), i = 0..7, without overflow
        const int w = b - a, w9 = w / 9, r9 = w % 9;
        int c = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            c += ci[a + (i + 1) * w9 + ((i + 1) * r9) / 9] < key ? 1 : 0;
        const int na = c == 0 ? a : a + c * w9 + (c * r9) / 9 + 1;
        const int nb = c == 8 ? b : a + (c + 1) * w9 + ((c + 1) * r9) / 9;
        a = na;
        b = nb;
    }
    int c = 0;
    if (b > a) {  // the last (at most 8) loaded together, clamped to the range
        int v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ci[a + i < b ? a + i : b - 1];
#pragma unroll
        for (int i = 0; i < 8; ++i) c += (a + i < b && v[i] < key) ? 1 : 0;
    }
    return a + c;
}

// Per row: starts[b][r] (relative to the row) and the counts cnt[b][r] (the
// virtual entry in its block), and with vdiag the virtual entry's position
// ins[r] (the first column >= r, kept inside its block's run) and flags[1]
// for a diagonal.  A group of G lanes (G a power of two > nb) per row: lane
// b in 1..nb-1 searches the whole row for block b's start, lane nb for the
// virtual entry's place, and a running maximum over the group keeps the
// starts non-decreasing whatever the order (one search deep instead of nb
// in sequence: config E 95 -> 20 us).
template <int G>
__global__ __launch_bounds__(256) void rows_search_kernel(FlatSplit a, int32_t* __restrict__ cnt) {
    const int lane = threadIdx.x & 63;
    const int j = lane & (G - 1);
    const int64_t r = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / G;
    const bool live = r < a.n;
    const int lo = live ? a.rp[r] : 0, hi = live ? a.rp[r + 1] : 0;
    const int len = hi - lo;
    int sj = 0;
    if (live && j >= 1 && j < a.nb)
        sj = lower_bound_col(a.ci, lo, hi, static_cast<int64_t>(j) * a.rows_per_block) - lo;
    else if (live && j >= a.nb)
        sj = len;
    int ins = 0;
    if (live && a.vdiag && j == a.nb) ins = lower_bound_col(a.ci, lo, hi, r) - lo;
    // running maximum over the group's lanes 0..j (starts non-decreasing)
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
        const int v = __shfl_up(sj, o, G);
        if (j >= o) sj = sj > v ? sj : v;
    }
    const int next = __shfl_down(sj, 1, G);  // lane j + 1's start (lanes < nb)
    const int d = a.vdiag ? block_of(static_cast<int>(live ? r : 0), a) : -1;
    const int sd = __shfl(sj, d < 0 ? 0 : d, G), sd1 = __shfl(sj, d < 0 ? 0 : d + 1, G);
    ins = __shfl(ins, a.nb, G);
    if (!live) return;
    if (j < a.nb) {
        const int64_t t = static_cast<int64_t>(j) * a.n + r;
        const int e = j + 1 < a.nb ? next : len;
        a.starts[t] = sj;
        cnt[t] = e - sj + (j == d ? 1 : 0);
    }
    // rows past the per-row scatter's share, for the scatter's first workgroups
    if (j == 0 && len > kRowCap) a.long_rows[atomicAdd(&a.flags[3], 1)] = static_cast<int32_t>(r);
    if (a.vdiag && j == 0) {
        ins = ins < sd ? sd : (ins > sd1 ? sd1 : ins);
        a.ins[r] = ins;
        if (ins < len && a.ci[lo + ins] == r) atomicOr(&a.flags[1], 1);
    }
}

constexpr int kRowSU = 8;  // 64-entry slices in flight per wavefront

// Entries [kb, ke) of row r (entries [lo, hi)) to the copy: entry k of block
// b goes to obase[b][r] + k (one further past the virtual entry in its
// block).  Lane j < nb holds block j's base (ob) and start (st).  An entry's
// block is taken from its position among the row's block starts, not from
// its column: for a sorted row the two agree (the starts were searched in
// the same columns), an unsorted one is flagged, and either way every store
// lands in its (block, row) segment.  Column-derived blocks (a
// double-precision division and three lane shuffles per entry) measured the
// same.  `step`: the distance between this wavefront's slice groups.
//
// Each 64-entry slice finds the blocks of its first and last positions (a
// ballot of the starts at or before them), and lanes compare their
// positions only with the starts inside the slice (a slice in one block:
// none).  The virtual entry's shift is positional too: in block d (the
// diagonal's), the entries from ins[r] (the first column >= r, clamped to
// the block's run) to the block's end, which for a sorted row without a
// diagonal are those of columns > r.  The predecessor column (the order
// check) comes from a wavefront shift.  (Lanes counting every start made
// the pass VALU-bound: about 55 vector instructions per slice, config E's
// A + I 0.19 ms of the scatter.)  Every lane of the wavefront calls it with
// the same row (r, lo, hi, kb, ke uniform).
__device__ __forceinline__ void scatter_range(const FlatSplit& a, int64_t r, int lo, int hi,
                                              int kb, int ke, int step, int ob, int st,
                                              int lane) {
    constexpr int kNone = 0x7FFFFFFF;
    const int row = static_cast<int>(r);
    const int R = a.rows_per_block;
    // positions [ins_lo, ins_lo + ins_n) move up one (the virtual entry's
    // block from the virtual entry on); ins_n = 0: none
    int ins_lo = 0;
    unsigned ins_n = 0;
    if (a.vdiag) {
        const int d = block_of(row, a);
        ins_lo = a.ins[r];
        const int e = __builtin_amdgcn_readlane(st, d + 1);  // d + 1 <= nb < 64
        ins_n = static_cast<unsigned>((e == kNone ? hi - lo : e) - ins_lo);
    }
    for (int k0 = kb; k0 < ke; k0 += step) {
        const int kend = k0 + 64 * kRowSU < ke ? k0 + 64 * kRowSU : ke;
        int c[kRowSU];
        float x[kRowSU];
#pragma unroll
        for (int u = 0; u < kRowSU; ++u) {
            const int k = k0 + u * 64 + lane;
            c[u] = k < kend ? a.ci[k] : 0;
            x[u] = (a.bv && k < kend) ? a.v[k] : 0.0f;
        }
        // the column before the group (its first entry's predecessor)
        int carry = k0 > lo ? a.ci[k0 - 1] : 0;
#pragma unroll
        for (int u = 0; u < kRowSU; ++u) {
            const int ks = k0 + u * 64;  // the slice's first entry
            if (ks >= kend) break;
            const int k = ks + lane;
            const int kr = k - lo;
            // every lane takes part in the shift and the read (lanes past
            // the end included)
            const int pc = __builtin_amdgcn_update_dpp(carry, c[u], 0x138 /* wave_shr:1 */, 0xF,
                                                       0xF, false);
            carry = __builtin_amdgcn_readlane(c[u], 63);
            // the blocks of the slice's first and last positions: the starts
            // 1.. at or before them (lane j holds block j's start)
            const int f = ks - lo, l = f + 63;
            const int bl = __popcll(__ballot(st <= f) & ~1ull);
            const int bh = __popcll(__ballot(st <= l) & ~1ull);
            int base = __builtin_amdgcn_readlane(ob, bl);
            int boff = bl * R;
            for (int j = bl + 1; j <= bh; ++j) {  // starts inside the slice
                const bool past = kr >= __builtin_amdgcn_readlane(st, j);
                base = past ? __builtin_amdgcn_readlane(ob, j) : base;
                boff = past ? j * R : boff;
            }
            if (k < kend) {
                const int c0 = c[u];
                if (kr > 0 && pc > c0) atomicOr(&a.flags[0], 1);
                if (a.vdiag && c0 == row) atomicOr(&a.flags[1], 1);
                const unsigned o = static_cast<unsigned>(base + k) +
                                   (static_cast<unsigned>(kr - ins_lo) < ins_n ? 1u : 0u);
                if (a.bci16)
                    a.bci16[o] = static_cast<uint16_t>(c0 - boff);
                else
                    a.bci[o] = c0;
                if (a.bv) a.bv[o] = x[u];
            }
        }
    }
}

// Row r's block bases and starts, lane j < nb.
__device__ __forceinline__ void row_blocks(const FlatSplit& a, int64_t r, int lane, int& ob,
                                           int& st) {
    ob = 0;
    st = 0x7FFFFFFF;  // (no block: after every entry)
    if (lane < a.nb) {
        const int64_t t = static_cast<int64_t>(lane) * a.n + r;
        ob = a.obase[t];
        st = a.starts[t];
    }
}

// The scatter, one launch.  Workgroups kLongWgs and above: one wavefront
// per row, its first kRowCap entries (one wavefront walking a 20,000-entry
// row alone bounded the whole pass: config E's A + I 0.37 ms).  The first
// kLongWgs workgroups: the rest of every row longer than kRowCap (rows
// a.long_rows[0 .. flags[3]), taken in turn), the four wavefronts of a
// workgroup taking the row's slice groups in turn.  Launched first, they run
// beside the per-row part (a launch of their own after it: 0.14 ms of
// config E's 0.33 ms scatter).
__global__ __launch_bounds__(256) void rows_scatter_kernel(FlatSplit a) {
    const int lane = threadIdx.x & 63;
    // the wavefront's index, uniform (and so its row, bounds and slices)
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    int ob, st;
    if (blockIdx.x < kLongWgs) {
        const int count = a.flags[3];
        for (int i = blockIdx.x; i < count; i += kLongWgs) {
            const int64_t r = a.long_rows[i];
            const int lo = a.rp[r], hi = a.rp[r + 1];
            row_blocks(a, r, lane, ob, st);
            scatter_range(a, r, lo, hi, lo + kRowCap + w * 64 * kRowSU, hi,
                               4 * 64 * kRowSU, ob, st, lane);
        }
        return;
    }
    const int64_t r = static_cast<int64_t>(blockIdx.x - kLongWgs) * 4 + w;
    if (r >= a.n) return;  // uniform per wave
    const int lo = a.rp[r], hi = a.rp[r + 1];
    row_blocks(a, r, lane, ob, st);
    const int ke = hi - lo > kRowCap ? lo + kRowCap : hi;
    scatter_range(a, r, lo, hi, lo, ke, 64 * kRowSU, ob, st, lane);
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

// The split's temporaries: counts (then the flat split's output bases),
// the scans' temp, flags ([0] out of block order, [1] a diagonal (vdiag),
// [2] the general split's disorder), and the flat split's row-start bitmap,
// slice ranks, non-empty rows, run starts and virtual-entry positions.
struct SplitTemps {
    int32_t *cnt, *flags, *starts, *ins, *nonempty, *nzrank, *nz_rows, *popc, *slice_rank;
    uint64_t* bits;
    int64_t* scan_tmp;
};

SplitTemps carve_split(Carver& c, int64_t n, int64_t nnz_src, int64_t nb) {
    const int64_t slices = ceil_div(std::max<int64_t>(nnz_src, 1), 64);
    SplitTemps t;
    t.bits = c.take<uint64_t>(slices);
    t.cnt = c.take<int32_t>(nb * n);
    t.scan_tmp = c.take<int64_t>(scan_temp_elems(std::max(nb * n, slices)));
    t.flags = c.take<int32_t>(4);
    t.starts = c.take<int32_t>(nb * n);
    t.ins = c.take<int32_t>(n);
    t.nonempty = c.take<int32_t>(n);
    t.nzrank = c.take<int32_t>(n + 1);
    t.nz_rows = c.take<int32_t>(n);
    t.popc = c.take<int32_t>(slices);
    t.slice_rank = c.take<int32_t>(slices + 1);
    return t;
}

// Shapes the blocked copy for n rows and nnz entries and returns its
// temporaries.
SplitTemps setup_blocked(BlockedCSR& bk, int64_t n, int64_t nnz, int64_t nnz_src,
                         const int32_t* rp, bool weighted, int64_t rows_per_block) {
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
    // 64 bytes past the indices: the 16-bit passes' scalar loads read whole
    // 16-entry batches, up to 15 entries past a chunk's end
    bk.bci.reserve(static_cast<size_t>(std::max<int64_t>(nnz, 1)) *
                       (bk.idx16 ? sizeof(uint16_t) : sizeof(int32_t)) +
                   64);
    if (weighted) bk.bv.reserve(static_cast<size_t>(std::max<int64_t>(nnz, 1)) * sizeof(float));
    Carver cv(nullptr, 0);
    carve_split(cv, n, nnz_src, nb);
    bk.scratch.reserve(cv.bytes());
    Carver c(bk.scratch.get(), bk.scratch.size());
    // host results: the plans' totals (4 per block), then the flags
    bk.host.reserve(static_cast<size_t>(4 * nb + 2) * sizeof(int64_t));
    bk.plans.resize(static_cast<size_t>(nb));
    for (auto& p : bk.plans)
        if (!p) p = std::make_unique<tg_spmm_plan_s>();
    return carve_split(c, n, nnz_src, nb);
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
    if (bk.resident) build_resident_split(bk, max_f, s);
    else bk.resident_wgs = 0;
}

// The caller's after_split hook, once.
void fire_after_split(BlockedCSR& bk) {
    if (!bk.after_split) return;
    std::function<void()> f = std::move(bk.after_split);
    bk.after_split = nullptr;
    f();
}

// The flat split (with or without the virtual diagonal); false when some
// row is out of block order or, with vdiag, has a diagonal (the copy is
// then incomplete and the caller takes another path).
bool split_flat(BlockedCSR& bk, const SplitTemps& t, const int32_t* rp, const int32_t* ci,
                const float* v, int64_t nnz_src, bool vdiag, int64_t max_f, int64_t chunk,
                hipStream_t s) {
    const int64_t n = bk.n, nb = bk.n_blocks;
    const int64_t slices = ceil_div(std::max<int64_t>(nnz_src, 1), 64);
    auto grid = [](int64_t x) { return static_cast<unsigned>(ceil_div(std::max<int64_t>(x, 1), 256)); };
    fill_i32(t.flags, 4, 0, s);
    fill_i32(reinterpret_cast<int32_t*>(t.bits), 2 * slices, 0, s);
    FlatSplit a{};
    a.rp = rp;
    a.ci = ci;
    a.v = v;
    a.n = n;
    a.nnz = nnz_src;
    a.rows_per_block = static_cast<int>(bk.rows_per_block);
    a.inv_rows = 1.0 / static_cast<double>(bk.rows_per_block);
    a.nb = static_cast<int>(nb);
    a.vdiag = vdiag ? 1 : 0;
    a.bits = t.bits;
    a.slice_rank = t.slice_rank;
    a.nz_rows = t.nz_rows;
    a.starts = t.starts;
    a.ins = t.ins;
    a.flags = t.flags;
    flat_marks_kernel<<<grid(n), 256, 0, s>>>(a, reinterpret_cast<uint32_t*>(t.bits), t.nonempty);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(t.nonempty, t.nzrank, n, t.scan_tmp, s);
    flat_nzrows_kernel<<<grid(n), 256, 0, s>>>(rp, n, t.nzrank, t.nz_rows);
    TG_LAUNCH_CHECK();
    flat_popc_kernel<<<grid(slices), 256, 0, s>>>(t.bits, slices, t.popc);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(t.popc, t.slice_rank, slices, t.scan_tmp, s);
    // waves of kFlatSU slices, four per workgroup
    const unsigned egrid = static_cast<unsigned>(ceil_div(slices, 4 * kFlatSU));
    if (nnz_src > 0) {
        flat_count_kernel<<<egrid, 256, 0, s>>>(a);
        TG_LAUNCH_CHECK();
    }
    flat_counts_kernel<<<grid(n * nb), 256, 0, s>>>(a, t.cnt);
    TG_LAUNCH_CHECK();
    int32_t* brp = bk.brp.as<int32_t>();
    exclusive_scan_i32(t.cnt, brp, nb * n, t.scan_tmp, s);
    flat_bases_kernel<<<grid(n * nb), 256, 0, s>>>(a, brp, t.cnt);
    TG_LAUNCH_CHECK();
    a.obase = t.cnt;
    a.bci = bk.idx16 ? nullptr : bk.bci.as<int32_t>();
    a.bci16 = bk.idx16 ? bk.bci.as<uint16_t>() : nullptr;
    a.bv = v ? bk.bv.as<float>() : nullptr;
    if (nnz_src > 0) {
        flat_scatter_kernel<<<egrid, 256, 0, s>>>(a);
        TG_LAUNCH_CHECK();
    }
    fire_after_split(bk);
    if (vdiag) {
        flat_diag_kernel<<<grid(n), 256, 0, s>>>(a, brp);
        TG_LAUNCH_CHECK();
    }
    int32_t* hf = reinterpret_cast<int32_t*>(bk.host.as<int64_t>() + 4 * nb);
    TG_HIP(hipMemcpyAsync(hf, t.flags, 2 * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    build_block_plans(bk, max_f, chunk, s);
    return hf[0] == 0 && hf[1] == 0;
}

// The row split (long sorted rows; with or without the virtual diagonal);
// false as split_flat.
bool split_rows(BlockedCSR& bk, const SplitTemps& t, const int32_t* rp, const int32_t* ci,
                const float* v, int64_t nnz_src, bool vdiag, int64_t max_f, int64_t chunk,
                hipStream_t s) {
    const int64_t n = bk.n, nb = bk.n_blocks;
    auto grid = [](int64_t x) { return static_cast<unsigned>(ceil_div(std::max<int64_t>(x, 1), 256)); };
    fill_i32(t.flags, 4, 0, s);
    FlatSplit a{};
    a.rp = rp;
    a.ci = ci;
    a.v = v;
    a.n = n;
    a.nnz = nnz_src;
    a.rows_per_block = static_cast<int>(bk.rows_per_block);
    a.inv_rows = 1.0 / static_cast<double>(bk.rows_per_block);
    a.nb = static_cast<int>(nb);
    a.vdiag = vdiag ? 1 : 0;
    a.starts = t.starts;
    a.ins = t.ins;
    a.flags = t.flags;
    a.long_rows = t.nz_rows;  // (the flat split's non-empty-row list, unused here)
    // a group of G lanes per row, G the power of two above nb
    const int g = nb < 2 ? 2 : nb < 4 ? 4 : nb < 8 ? 8 : nb < 16 ? 16 : nb < 32 ? 32 : 64;
    require(nb < 64, "blocked CSR: the row split takes at most 63 blocks");
    const unsigned sgrid = static_cast<unsigned>(ceil_div(n * g, 256));
    switch (g) {
        case 2: rows_search_kernel<2><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
        case 4: rows_search_kernel<4><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
        case 8: rows_search_kernel<8><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
        case 16: rows_search_kernel<16><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
        case 32: rows_search_kernel<32><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
        default: rows_search_kernel<64><<<sgrid, 256, 0, s>>>(a, t.cnt); break;
    }
    TG_LAUNCH_CHECK();
    int32_t* brp = bk.brp.as<int32_t>();
    exclusive_scan_i32(t.cnt, brp, nb * n, t.scan_tmp, s);
    flat_bases_kernel<<<grid(n * nb), 256, 0, s>>>(a, brp, t.cnt);
    TG_LAUNCH_CHECK();
    a.obase = t.cnt;
    a.bci = bk.idx16 ? nullptr : bk.bci.as<int32_t>();
    a.bci16 = bk.idx16 ? bk.bci.as<uint16_t>() : nullptr;
    a.bv = v ? bk.bv.as<float>() : nullptr;
    if (nnz_src > 0) {
        // the long rows' workgroups first (their number stays on the device)
        const int64_t rgrid = kLongWgs + ceil_div(n, 4);
        require(rgrid < (int64_t(1) << 31), "blocked CSR: too many rows");
        rows_scatter_kernel<<<static_cast<unsigned>(rgrid), 256, 0, s>>>(a);
        TG_LAUNCH_CHECK();
    }
    fire_after_split(bk);
    if (vdiag) {
        flat_diag_kernel<<<grid(n), 256, 0, s>>>(a, brp);
        TG_LAUNCH_CHECK();
    }
    int32_t* hf = reinterpret_cast<int32_t*>(bk.host.as<int64_t>() + 4 * nb);
    TG_HIP(hipMemcpyAsync(hf, t.flags, 2 * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    build_block_plans(bk, max_f, chunk, s);
    return hf[0] == 0 && hf[1] == 0;
}

// Sorted-row splits: the row split for long rows, the flat one otherwise.
bool split_sorted(BlockedCSR& bk, const SplitTemps& t, const int32_t* rp, const int32_t* ci,
                  const float* v, int64_t nnz_src, bool vdiag, int64_t max_f, int64_t chunk,
                  hipStream_t s) {
    if (nnz_src >= kRowSplitMinAvg * bk.n && bk.n_blocks < 64)
        return split_rows(bk, t, rp, ci, v, nnz_src, vdiag, max_f, chunk, s);
    return split_flat(bk, t, rp, ci, v, nnz_src, vdiag, max_f, chunk, s);
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
    fire_after_split(bk);
    int32_t* hf = reinterpret_cast<int32_t*>(bk.host.as<int64_t>() + 4 * nb);
    TG_HIP(hipMemcpyAsync(hf, disorder, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    build_block_plans(bk, max_f, chunk, s);
    bk.in_order = hf[0] == 0;
}

}  // namespace

void build_blocked(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                   const int32_t* ci, const float* v, int64_t rows_per_block, int64_t max_f,
                   hipStream_t s, int64_t chunk) {
    const SplitTemps t = setup_blocked(bk, n, nnz, nnz, rp, v != nullptr, rows_per_block);
    require(nnz == 0 || ci != nullptr, "blocked CSR: null structure");
    bk.vdiag = false;
    // rows in block order (sorted rows) take the flat split; the general
    // one runs when some row is not
    if (split_sorted(bk, t, rp, ci, v, nnz, false, max_f, chunk, s)) {
        bk.in_order = true;
        return;
    }
    split_general(bk, t, rp, ci, v, max_f, chunk, s);
}

bool build_blocked_self_loops(BlockedCSR& bk, int64_t n, int64_t nnz, const int32_t* rp,
                              const int32_t* ci, int64_t rows_per_block, int64_t max_f,
                              hipStream_t s, int64_t chunk) {
    require(nnz + n < (int64_t(1) << 31), "blocked CSR: nnz + n must be < 2^31");
    const SplitTemps t = setup_blocked(bk, n, nnz + n, nnz, rp, false, rows_per_block);
    require(nnz == 0 || ci != nullptr, "blocked CSR: null structure");
    bk.vdiag = true;
    if (!split_sorted(bk, t, rp, ci, nullptr, nnz, true, max_f, chunk, s)) return false;
    bk.in_order = true;
    return true;
}

namespace {

// The resident passes' row ranges: range w starts near the row where the
// running count of the copy's entries (rp[r], plus r for the rows'
// diagonals when the split placed them: the same counts for both ways of
// building A + I's copy) reaches w/W of the total, then one thread walks the
// W bounds so that every range holds at most `cap` rows (n <= W * cap).
__global__ __launch_bounds__(1024) void resident_split_kernel(const int32_t* __restrict__ rp,
                                                              int64_t n, int vdiag, int W,
                                                              int cap,
                                                              int32_t* __restrict__ wg_rows) {
    __shared__ int32_t lb[1024];
    const int w = threadIdx.x;
    const int64_t tot = static_cast<int64_t>(rp[n]) + (vdiag ? n : 0);
    if (w <= W) {
        const int64_t target = tot * w / W;
        int64_t lo = 0, hi = n;  // the first r whose count reaches target
        while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (static_cast<int64_t>(rp[mid]) + (vdiag ? mid : 0) < target) lo = mid + 1;
            else hi = mid;
        }
        lb[w] = static_cast<int32_t>(lo);
    }
    __syncthreads();
    if (w == 0) {
        int64_t prev = 0;
        lb[0] = 0;
        for (int k = 1; k < W; ++k) {
            int64_t e = lb[k];
            e = e < prev ? prev : e;
            e = e > prev + cap ? prev + cap : e;
            const int64_t need = n - static_cast<int64_t>(W - k) * cap;
            e = e < need ? need : e;
            lb[k] = static_cast<int32_t>(e);
            prev = e;
        }
        lb[W] = static_cast<int32_t>(n);
    }
    __syncthreads();
    if (w <= W) wg_rows[w] = lb[w];
}

}  // namespace

void build_resident_split(BlockedCSR& bk, int64_t max_f, hipStream_t s) {
    bk.resident_wgs = 0;
    if (!bk.idx16 || bk.weighted || bk.n <= 0) return;
    int dev = 0, cus = 0;
    TG_HIP(hipGetDevice(&dev));
    TG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t W = std::min<int64_t>(std::min<int64_t>(kResidentPerCU * cus, 1023), bk.n);
    if (W <= 0 || bk.n > W * kResidentRows) return;
    bk.wg_rows.reserve(static_cast<size_t>(W + 1) * sizeof(int32_t));
    resident_split_kernel<<<1, 1024, 0, s>>>(bk.rp, bk.n, bk.vdiag ? 1 : 0, static_cast<int>(W),
                                             kResidentRows, bk.wg_rows.as<int32_t>());
    TG_LAUNCH_CHECK();
    bk.max_phases = ceil_div(std::max<int64_t>(max_f, 1), 32) * bk.n_blocks;
    bk.phase_count.reserve(static_cast<size_t>(bk.max_phases) * sizeof(int32_t));
    bk.resident_wgs = W;
}

void run_aggregate_blocked(const BlockedCSR& bk, int64_t f, const float* b, int64_t ldb,
                           float* c, int64_t ldc, const AggEpilogue& epi, hipStream_t s) {
    require(!epi.max, "blocked aggregation: max is not supported");
    require(!epi.acc && !epi.skip_empty, "blocked aggregation: pass flags are set per block");
    if (bk.n == 0 || f == 0) return;
    if (resident_ok(bk, f, b, ldb, epi)) return run_aggregate_resident(bk, f, b, ldb, c, ldc, epi, s);
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
        e.mask_tail = epi.mask_tail;
        e.att_src = epi.att_src;
        e.att_dst = epi.att_dst;
        e.att_max = epi.att_max;
        e.att_rinv = epi.att_rinv;
        e.att_heads = epi.att_heads;
        e.att_slope = epi.att_slope;
        // 16-bit indices count from the block's first source row
        const int64_t r0 = bk.idx16 ? blk * bk.rows_per_block : 0;
        const float* bb = b + r0 * (epi.b_tile_stride > 0 ? 32 : ldb);
        // (the buffer gathers' column 0xFFFF must lie past every block)
        e.b_rows = bk.idx16 && bk.rows_per_block <= 65535 ? bk.n - r0 : 0;
        if (bk.idx16) {
            e.ci16 = bk.bci.as<uint16_t>();
            if (e.att_dst) e.att_dst = epi.att_dst + r0 * epi.att_heads;
        }
        run_aggregate(*bk.plans[blk], f, bci, bv, bb, ldb, c, ldc, e, s, group_cols);
    }
}

}  // namespace tg
