// gat.hip -- multi-head GAT on gfx950.
//
// Replaces GATLayer::forward (reference src/layers.cpp:945-1129) run once
// per head, and Model's head concat / average (src/model.cpp:312-354,
// :403-421), for all heads of a layer at once:
//   * Wh = H * [W_0 | W_1 | ...] is one GEMM (the caller's);
//   * gat_scores: src[i,h] = a_l(h).Wh_i(h), dst[i,h] = a_r(h).Wh_i(h) in
//     the reference's operation order (8 interleaved fma partial sums, then
//     the lane sum, then the tail; layers.cpp:991-1026);
//   * gat_chunk_kernel, one pass per row chunk of the degree-binned plan:
//     each lane scores e_ij = LeakyReLU(src_i + dst_j) for the head of its
//     feature vector and keeps an online softmax -- running max, running
//     sum of exp(e - max), and the accumulated exp(e - max) * Wh_j(h),
//     rescaled when the max grows -- so the row is read once; the store
//     multiplies by 1/sum, giving the reference's
//     out_i = sum_j exp(e_ij - max) (1/sum) Wh_j (layers.cpp:1076-1109).
//     The nnz x heads attention matrix is never stored.  Bias, the layer
//     activation and the model's post activation are applied on store.
//   * rows longer than one chunk: every chunk stores its unnormalised sum
//     with its own (max, sum); gat_reduce_kernel merges them in chunk order
//     (max of maxima, sums rescaled by exp(m_c - M)).
//   * column-blocked form (large, dense graphs), fast precision: the online
//     softmax carried across the block passes (gat_online_chunk_kernel, a
//     running max and sum per row and column group), where a lane group
//     holding a whole head computes dst_j = a_r . Wh_j from the rows it
//     gathers instead of reading it; exact precision and the other layouts:
//     a statistics sweep (gat_exact_stats_kernel / gat_stats_kernel: each
//     row's max score and 1/sum per head), then passes (blocked.hip) that
//     compute alpha_ij = exp(e_ij - max_i) * (1/sum_i) per entry and head from
//     the [n x heads] scores and statistics (the attention mode of the
//     aggregation kernel).  The attention matrix is never stored here either.
#include "aggregate.hpp"
#include "common.hpp"
#include "device_utils.hpp"
#include "spmm_plan.hpp"

#include <string>

namespace tg {

// (m, s) per partial slot and head, or per 32-column group (blocked online
// passes), whichever is more
int64_t gat_stat_slots(int64_t heads, int64_t f) {
    return std::max<int64_t>(heads, ceil_div(heads * f, 32));
}

namespace {

template <int VEC>
struct VecT;
template <>
struct VecT<1> { using T = float; };
template <>
struct VecT<2> { using T = float2; };
template <>
struct VecT<4> { using T = float4; };

template <int VEC>
__device__ __forceinline__ void ldv(const float* p, float (&x)[VEC]) {
    typename VecT<VEC>::T t = *reinterpret_cast<const typename VecT<VEC>::T*>(p);
    const float* q = reinterpret_cast<const float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = q[k];
}

template <int VEC>
__device__ __forceinline__ void stv(float* p, const float (&x)[VEC]) {
    typename VecT<VEC>::T t;
    float* q = reinterpret_cast<float*>(&t);
#pragma unroll
    for (int k = 0; k < VEC; ++k) q[k] = x[k];
    *reinterpret_cast<typename VecT<VEC>::T*>(p) = t;
}

__device__ __forceinline__ float lrelu(float e, float slope) { return (e >= 0.0f) ? e : slope * e; }


__device__ __forceinline__ float finish_val(float x, const float* bias, int64_t fo, int act,
                                            int post, bool exact = false) {
    if (bias) x = x + bias[fo];
    if (act == TG_ACT_RELU) x = (0.0f < x) ? x : 0.0f;
    if (post == TG_POST_RELU) {
        x = (0.0f < x) ? x : 0.0f;
    } else if (post == TG_POST_ELU) {
        if (x < 0.0f) x = 1.0f * ((exact ? exp_rn(x) : expf(x)) - 1.0f);
    }
    return x;
}

__global__ __launch_bounds__(256) void gat_scores_kernel(int64_t n, int heads, int f,
                                                         const float* __restrict__ wh,
                                                         int64_t ldwh,
                                                         const float* __restrict__ al,
                                                         const float* __restrict__ ar,
                                                         float* __restrict__ src,
                                                         float* __restrict__ dst) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * heads) return;
    const int64_t i = t / heads;
    const int h = static_cast<int>(t % heads);
    const float* w = wh + i * ldwh + static_cast<int64_t>(h) * f;
    const float* a = al + static_cast<int64_t>(h) * f;
    const float* b = ar + static_cast<int64_t>(h) * f;
    const int f8 = (f / 8) * 8;
    float ls[8], ld[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) ls[l] = ld[l] = 0.0f;
    for (int q = 0; q < f8; q += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float x = w[q + l];
            ls[l] = __builtin_fmaf(a[q + l], x, ls[l]);
            ld[l] = __builtin_fmaf(b[q + l], x, ld[l]);
        }
    }
    float s = 0.0f, d = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        s = s + ls[l];
        d = d + ld[l];
    }
    // Tail: groups of four as separate multiply and add, the rest fused
    // (the operation sequence of the reference's compiled scalar tail).
    const int t4 = f8 + ((f - f8) / 4) * 4;
    for (int q = f8; q < t4; ++q) {
        s = s + a[q] * w[q];
        d = d + b[q] * w[q];
    }
    for (int q = t4; q < f; ++q) {
        s = __builtin_fmaf(a[q], w[q], s);
        d = __builtin_fmaf(b[q], w[q], d);
    }
    src[t] = s;
    dst[t] = d;
}

// gat_scores_kernel with the workgroup's Wh segments staged in LDS (f <= 64,
// f % 4 == 0 or one head with row padding to the next multiple of 4,
// 16-byte aligned rows, heads <= 16: at most 41.6 KB): 128
// (node, head) pairs per workgroup,
// their segments read with coalesced 128-bit loads (a thread's own 64-float
// segment read by itself scatters every load over 64 lines: config E's
// layer-1 scores 95 µs, 2.5 TB/s of Wh) into rows of f + 1 floats, so that
// the threads' reads of their own rows fall in distinct banks; a_l and a_r
// likewise.  Then every thread runs the same operations in the same order.
constexpr int kScorePairs = 128;

__global__ __launch_bounds__(kScorePairs) void gat_scores_lds_kernel(
    int64_t n, int heads, int f, const float* __restrict__ wh, int64_t ldwh,
    const float* __restrict__ al, const float* __restrict__ ar, float* __restrict__ src,
    float* __restrict__ dst) {
    extern __shared__ float sm[];  // [kScorePairs][fp], then a_l, a_r: [heads][fp]
    // a segment of f4 128-bit vectors (one head whose f is not a multiple
    // of 4: its last vector runs into the row's padding, loaded, never used)
    const int f4 = (f + 3) / 4;
    const int fp = 4 * f4 + 1;
    float* sa = sm + kScorePairs * fp;
    float* sb = sa + heads * fp;
    const int64_t total = n * heads;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kScorePairs;
    const int np = static_cast<int>(total - p0 < kScorePairs ? total - p0 : kScorePairs);
    // the pairs' segments (a segment's f floats are whole 128-bit vectors):
    // at most 16 vectors a thread, all loaded before the first store
    constexpr int kV = 16;  // kScorePairs * 64 / 4 / kScorePairs
    const int nv = np * f4;
    // x / d as (x * ceil(2^16 / d)) >> 16: exact for x < 4096 and d <= 16
    // (here x < 2048), where the division instructions dominated the loop
    const unsigned mf4 = (65536u + f4 - 1) / f4, mh = (65536u + heads - 1) / heads;
    const int64_t node0 = p0 / heads;
    const int r0 = static_cast<int>(p0 - node0 * heads);
    float4 xv[kV];
#pragma unroll
    for (int u = 0; u < kV; ++u) {
        const int e = threadIdx.x + u * kScorePairs;
        if (e < nv) {
            const int pl = static_cast<int>((static_cast<unsigned>(e) * mf4) >> 16);
            const int k = (e - pl * f4) * 4;
            const int q = r0 + pl;  // the pair's offset from node0's first head
            const int dn = static_cast<int>((static_cast<unsigned>(q) * mh) >> 16);
            const int h = q - dn * heads;
            xv[u] = *reinterpret_cast<const float4*>(wh + (node0 + dn) * ldwh + h * f + k);
        }
    }
#pragma unroll
    for (int u = 0; u < kV; ++u) {
        const int e = threadIdx.x + u * kScorePairs;
        if (e < nv) {
            const int pl = static_cast<int>((static_cast<unsigned>(e) * mf4) >> 16);
            const int k = (e - pl * f4) * 4;
            float* d = sm + pl * fp + k;
            d[0] = xv[u].x; d[1] = xv[u].y; d[2] = xv[u].z; d[3] = xv[u].w;
        }
    }
    for (int e = threadIdx.x; e < heads * f; e += kScorePairs) {
        const int h = e / f, k = e - h * f;
        sa[h * fp + k] = al[e];
        sb[h * fp + k] = ar[e];
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) >= np) return;
    const int64_t t = p0 + threadIdx.x;
    const int h = static_cast<int>(t % heads);
    const float* w = sm + threadIdx.x * fp;
    const float* a = sa + h * fp;
    const float* b = sb + h * fp;
    const int f8 = (f / 8) * 8;
    float ls[8], ld[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) ls[l] = ld[l] = 0.0f;
    for (int q = 0; q < f8; q += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float x = w[q + l];
            ls[l] = __builtin_fmaf(a[q + l], x, ls[l]);
            ld[l] = __builtin_fmaf(b[q + l], x, ld[l]);
        }
    }
    float s = 0.0f, d = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        s = s + ls[l];
        d = d + ld[l];
    }
    const int t4 = f8 + ((f - f8) / 4) * 4;
    for (int q = f8; q < t4; ++q) {
        s = s + a[q] * w[q];
        d = d + b[q] * w[q];
    }
    for (int q = t4; q < f; ++q) {
        s = __builtin_fmaf(a[q], w[q], s);
        d = __builtin_fmaf(b[q], w[q], d);
    }
    src[t] = s;
    dst[t] = d;
}

struct GatArgs {
    const int4* chunks;
    int64_t n_chunks;
    const int4* split;
    int64_t n_split;
    const int32_t* ci;
    const float* wh;
    int64_t ldwh;
    const float* src;  // [n x heads]
    const float* dst;  // [n x heads]
    int heads;
    int f;             // per-head width
    int64_t ftot;      // heads * f
    float slope;
    float* out;
    int64_t ldo;
    float* partials;   // [n_partials x ldp]
    int64_t ldp;       // ftot rounded up to the access width
    float* pstats;     // [n_partials x heads x 2] (max, sum)
    const float* bias;
    int act;
    int post;
    int vec_io;        // stores and bias loads are full, aligned vectors
    int exact;         // the reference's operation order (rows never split)
};

// Applies the epilogue and stores one lane vector of row `row`.
template <int VEC>
__device__ __forceinline__ void gat_store(const GatArgs& a, int64_t row, int64_t fo,
                                          float (&x)[VEC], float scale) {
    if (a.vec_io) {
#pragma unroll
        for (int k = 0; k < VEC; ++k)
            x[k] = finish_val(x[k] * scale, a.bias, fo + k, a.act, a.post, a.exact);
        stv<VEC>(a.out + row * a.ldo + fo, x);
        return;
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (fo + k >= a.ftot) break;
        a.out[row * a.ldo + fo + k] =
            finish_val(x[k] * scale, a.bias, fo + k, a.act, a.post, a.exact);
    }
}

// Exact variant (the plan never splits rows): per row and head, the
// reference's sequence (layers.cpp:1056-1109) -- e = LeakyReLU(s_i + d_j);
// the row max; t = exp(e - max) summed in nonzero order; alpha = t * (1/sum)
// (0 when the sum is 0); out = fma(alpha, Wh_j, out) in nonzero order.  Each
// lane walks the whole row for its own head, so every sum is sequential.
template <int VEC, int LPR, int VPL>
__global__ __launch_bounds__(256) void gat_exact_kernel(GatArgs a) {
    constexpr int GPB = 256 / LPR;
    constexpr int TILE = LPR * VPL * VEC;
    constexpr int U = 8;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (cid >= a.n_chunks) return;
    const int4 ch = a.chunks[cid];
    const int row = ch.x, b = ch.y, e = ch.z;
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    const int H = a.heads;
    const float* srow = a.src + static_cast<int64_t>(row) * H;
    int64_t fo[VPL], fl[VPL];
    bool ok[VPL];
    int hv[VPL];
    float si[VPL], m[VPL], sum[VPL], inv[VPL], acc[VPL][VEC];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        fo[v] = fbase + static_cast<int64_t>(l + v * LPR) * VEC;
        ok[v] = fo[v] < a.ftot;
        fl[v] = ok[v] ? fo[v] : fbase;  // the tile's first vector: in bounds, never stored
        hv[v] = ok[v] ? static_cast<int>(fo[v] / a.f) : 0;
        si[v] = srow[hv[v]];
        m[v] = -INFINITY;
        sum[v] = 0.0f;
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[v][k] = 0.0f;
    }
    // passes 1 and 2: the max, then the sequential sum of exp(e - max)
    for (int pass = 0; pass < 2; ++pass) {
        for (int base = b; base < e; base += LPR) {
            const int idx = base + l;
            const int cl = idx < e ? a.ci[idx] : 0;
            const int cnt = e - base < LPR ? e - base : LPR;
            for (int t = 0; t < cnt; ++t) {
                const int col = __shfl(cl, t, LPR);
#pragma unroll
                for (int v = 0; v < VPL; ++v) {
                    const float x = lrelu(si[v] + a.dst[static_cast<int64_t>(col) * H + hv[v]], a.slope);
                    if (pass == 0)
                        m[v] = (m[v] < x) ? x : m[v];
                    else
                        sum[v] += exp_rn(x - m[v]);
                }
            }
        }
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v) inv[v] = (sum[v] > 0.0f) ? 1.0f / sum[v] : 0.0f;
    // pass 3: alpha-weighted rows in nonzero order, U gathers in flight
    for (int base = b; base < e; base += LPR) {
        const int idx = base + l;
        const int cl = idx < e ? a.ci[idx] : 0;
        const int cnt = e - base < LPR ? e - base : LPR;
        for (int s0 = 0; s0 < cnt; s0 += U) {
            int col[U];
            float w[U][VPL][VEC], al[U][VPL];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int t = s0 + u < LPR ? s0 + u : LPR - 1;
                col[u] = __shfl(cl, t, LPR);
                const float* wr = a.wh + static_cast<int64_t>(col[u]) * a.ldwh;
#pragma unroll
                for (int v = 0; v < VPL; ++v) {
                    const float x = lrelu(si[v] + a.dst[static_cast<int64_t>(col[u]) * H + hv[v]], a.slope);
                    al[u][v] = exp_rn(x - m[v]) * inv[v];
                    ldv<VEC>(wr + fl[v], w[u][v]);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool valid = s0 + u < cnt;
#pragma unroll
                for (int v = 0; v < VPL; ++v)
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const float nx = __builtin_fmaf(al[u][v], w[u][v][k], acc[v][k]);
                        acc[v][k] = valid ? nx : acc[v][k];
                    }
            }
        }
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v)
        if (ok[v]) gat_store<VEC>(a, row, fo[v], acc[v], 1.0f);
}

template <int VEC, int LPR, int VPL>
__global__ __launch_bounds__(256) void gat_chunk_kernel(GatArgs a) {
    constexpr int GPB = 256 / LPR;
    constexpr int U = VPL <= 2 ? 8 : 4;  // gathers in flight per lane
    constexpr int TILE = LPR * VPL * VEC;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (cid >= a.n_chunks) return;
    const int4 ch = a.chunks[cid];
    const int row = ch.x, b = ch.y, e = ch.z;
    const bool split = ch.w >= 0;
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    const int H = a.heads;
    const float* srow = a.src + static_cast<int64_t>(row) * H;

    int64_t fo[VPL];
    bool ok[VPL];
    int hv[VPL];
    float si[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        fo[v] = fbase + static_cast<int64_t>(l + v * LPR) * VEC;
        ok[v] = fo[v] < a.ftot;
        hv[v] = ok[v] ? static_cast<int>(fo[v] / a.f) : 0;
        si[v] = srow[hv[v]];
    }

    // One pass with an online softmax per lane vector (its head): running
    // max m, running sum s of exp(e - m), and acc = sum exp(e - m) Wh_j; a
    // larger max rescales s and acc by exp(m_old - m_new) (exactly 1 when
    // the max is unchanged, 0 from the initial -inf).  Lanes of one head see
    // the same scores, so their (m, s) agree.
    float m[VPL], s[VPL], acc[VPL][VEC];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        m[v] = -INFINITY;
        s[v] = 0.0f;
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[v][k] = 0.0f;
    }

    // Batches of BE entries: each lane loads CPL consecutive column indices
    // with one coalesced access, the group broadcasts them with shuffles,
    // and U gathers are in flight per step (slots past the chunk's end read
    // row 0 and are not accumulated).
    constexpr int CPL = U > LPR ? U / LPR : 1;
    constexpr int BE = LPR * CPL;
    for (int base = b; base < e; base += BE) {
        int cl[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int idx = base + l * CPL + j;
            cl[j] = idx < e ? a.ci[idx] : 0;
        }
        const int cnt = e - base < BE ? e - base : BE;
#pragma unroll
        for (int s0 = 0; s0 < BE; s0 += U) {
          if (s0 < cnt) {  // uniform across the group: no early exit in the unrolled body
            const int nv = cnt - s0 < U ? cnt - s0 : U;  // valid slots of this step
            int col[U];
#pragma unroll
            for (int u = 0; u < U; ++u) col[u] = __shfl(cl[(s0 + u) % CPL], (s0 + u) / CPL, LPR);
            float w[U][VPL][VEC];
            float ev[U][VPL];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float* wr = a.wh + static_cast<int64_t>(col[u]) * a.ldwh;
#pragma unroll
                for (int v = 0; v < VPL; ++v) {
                    ev[u][v] = a.dst[static_cast<int64_t>(col[u]) * H + hv[v]];
                    // lanes past ftot load the tile's first vector, never stored
                    ldv<VEC>(wr + (ok[v] ? fo[v] : fbase), w[u][v]);
                }
            }
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
                float mn = m[v];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    ev[u][v] = lrelu(si[v] + ev[u][v], a.slope);
                    if (u < nv) mn = (mn < ev[u][v]) ? ev[u][v] : mn;
                }
                const float sc = expf(m[v] - mn);
                m[v] = mn;
                s[v] *= sc;
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[v][k] *= sc;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const bool valid = u < nv;  // a select, not a branch
                    const float p = expf(ev[u][v] - mn);
                    s[v] = valid ? s[v] + p : s[v];
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const float nx = __builtin_fmaf(p, w[u][v][k], acc[v][k]);
                        acc[v][k] = valid ? nx : acc[v][k];
                    }
                }
            }
          }
        }
    }

    if (split) {
        // the chunk's (max, sum) per head, written by the lane that owns the
        // head's first feature
        float* prow = a.partials + static_cast<int64_t>(ch.w) * a.ldp;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            if (!ok[v]) continue;
            stv<VEC>(prow + fo[v], acc[v]);
            if (fo[v] % a.f == 0) {
                float* st = a.pstats + (static_cast<int64_t>(ch.w) * H + hv[v]) * 2;
                st[0] = m[v];
                st[1] = s[v];
            }
        }
        return;
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        if (!ok[v]) continue;
        // empty rows: s = 0 gives 0 before the bias (layers.cpp:1059)
        const float inv = (s[v] > 0.0f) ? 1.0f / s[v] : 0.0f;
        gat_store<VEC>(a, row, fo[v], acc[v], inv);
    }
}

template <int VEC, int LPR, int VPL>
__global__ __launch_bounds__(256) void gat_reduce_kernel(GatArgs a) {
    constexpr int GPB = 256 / LPR;
    constexpr int TILE = LPR * VPL * VEC;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t sid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (sid >= a.n_split) return;
    const int4 sp = a.split[sid];
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    const int H = a.heads;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        const int64_t fo = fbase + static_cast<int64_t>(l + v * LPR) * VEC;
        if (fo >= a.ftot) continue;
        const int h = static_cast<int>(fo / a.f);
        float M = -INFINITY;
        for (int c = 0; c < sp.z; ++c) {
            const float m = a.pstats[(static_cast<int64_t>(sp.y + c) * H + h) * 2];
            M = (M < m) ? m : M;
        }
        float S = 0.0f;
        float acc[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] = 0.0f;
        for (int c = 0; c < sp.z; ++c) {
            const float* st = a.pstats + (static_cast<int64_t>(sp.y + c) * H + h) * 2;
            const float sc = expf(st[0] - M);
            S = __builtin_fmaf(st[1], sc, S);
            float t[VEC];
            ldv<VEC>(a.partials + static_cast<int64_t>(sp.y + c) * a.ldp + fo, t);
#pragma unroll
            for (int k = 0; k < VEC; ++k) acc[k] = __builtin_fmaf(t[k], sc, acc[k]);
        }
        const float inv = (S > 0.0f) ? 1.0f / S : 0.0f;
        gat_store<VEC>(a, sp.x, fo, acc, inv);
    }
}

// Head average (concat = false): out = (sum over heads in order) * (1/heads),
// then the post activation (model.cpp:335-354, :426-435).
__global__ __launch_bounds__(256) void gat_average_kernel(const float* __restrict__ x,
                                                          int64_t n, int heads, int f,
                                                          float* __restrict__ out, int64_t ldo,
                                                          int post, int exact) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * f) return;
    const int64_t i = t / f, j = t % f;
    const float* xr = x + i * static_cast<int64_t>(heads) * f;
    float s = 0.0f;
    for (int h = 0; h < heads; ++h) s += xr[static_cast<int64_t>(h) * f + j];
    s *= 1.0f / static_cast<float>(heads);
    out[i * ldo + j] = finish_val(s, nullptr, 0, TG_ACT_NONE, post, exact != 0);
}

template <int VEC, int LPR, int VPL>
void launch_gat(const tg_spmm_plan_s& p, const LaneLayout& L, GatArgs& a, hipStream_t s) {
    constexpr int GPB = 256 / LPR;
    if (a.exact) {
        require(p.n_split == 0, "GATLayer: the exact edge pass needs a plan without split rows");
        if (p.n_chunks > 0) {
            dim3 grid(static_cast<unsigned>(ceil_div(p.n_chunks, GPB)),
                      static_cast<unsigned>(L.n_tiles));
            gat_exact_kernel<VEC, LPR, VPL><<<grid, 256, 0, s>>>(a);
            TG_LAUNCH_CHECK();
        }
        return;
    }
    if (p.n_chunks > 0) {
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_chunks, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        gat_chunk_kernel<VEC, LPR, VPL><<<grid, 256, 0, s>>>(a);
        TG_LAUNCH_CHECK();
    }
    if (p.n_split > 0) {
        dim3 grid(static_cast<unsigned>(ceil_div(p.n_split, GPB)),
                  static_cast<unsigned>(L.n_tiles));
        gat_reduce_kernel<VEC, LPR, VPL><<<grid, 256, 0, s>>>(a);
        TG_LAUNCH_CHECK();
    }
}

template <int VEC>
void dispatch_gat(const tg_spmm_plan_s& p, const LaneLayout& L, GatArgs& a, hipStream_t s) {
#define TG_GAT_CASE(LPR_, VPL_) \
    if (L.lpr == LPR_ && L.vpl == VPL_) return launch_gat<VEC, LPR_, VPL_>(p, L, a, s);
    TG_GAT_CASE(4, 1)
    TG_GAT_CASE(8, 1)
    TG_GAT_CASE(16, 1)
    TG_GAT_CASE(32, 1)
    TG_GAT_CASE(64, 1)
#undef TG_GAT_CASE
    throw std::logic_error("gat: no kernel for this lane layout");
}

// Merges two (max, sum of exp(e - max)) pairs of one head; -inf maxima
// carry an empty sum.
__device__ __forceinline__ void softmax_merge(float& m, float& s, float mo, float so) {
    const float M = (m < mo) ? mo : m;
    const float a = (m == -INFINITY) ? 0.0f : s * expf(m - M);
    const float c = (mo == -INFINITY) ? 0.0f : so * expf(mo - M);
    m = M;
    s = a + c;
}

// dst_j's values for the NH heads h0.. (NH = 4: one 16-byte load).
template <int NH>
__device__ __forceinline__ void gat_dst(const float* __restrict__ dst, int heads, int h0,
                                        int col, float (&d)[NH]) {
    const float* dj = dst + static_cast<int64_t>(col) * heads + h0;
    if constexpr (NH == 4) {
        const float4 t = *reinterpret_cast<const float4*>(dj);
        d[0] = t.x;
        d[1] = t.y;
        d[2] = t.z;
        d[3] = t.w;
    } else {
#pragma unroll
        for (int k = 0; k < NH; ++k) d[k] = dj[k];
    }
}

// One group of GL lanes per plan chunk (at most `chunk` entries of one
// row; GL = 64: a wave, 16 or 32: several chunks per wave), heads in groups
// of NH (4: heads in fours with 16-byte aligned dst; else 1), one sweep
// over the chunk: each lane takes four entries at a time, computes
// their scores e_ij = LeakyReLU(src_i + dst_j), raises its running max to
// the batch's maximum (rescaling its running sum once per batch) and adds
// exp(e - max) for the batch -- one L2 request per entry and head group,
// which bounds this kernel.  The lanes' (max, sum) pairs are merged by a
// butterfly (commutative merges: every lane ends with the same values).  A
// whole row writes its max and 1/sum (0 for an empty row, as the
// reference's zero sum gives a zero row before the bias); a split row's
// chunk writes its (max, sum) pair to its partial slot for
// gat_stats_merge_kernel.
template <int NH, int GL>
__global__ __launch_bounds__(256) void gat_stats_kernel(const int4* __restrict__ chunks,
                                                        int64_t n_chunks,
                                                        const int32_t* __restrict__ ci,
                                                        int heads,
                                                        const float* __restrict__ src,
                                                        const float* __restrict__ dst,
                                                        float slope, float* __restrict__ rmax,
                                                        float* __restrict__ rinv,
                                                        float* __restrict__ pstats) {
    const int lane = threadIdx.x % GL;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * (256 / GL) + threadIdx.x / GL;
    if (cid >= n_chunks) return;  // uniform per group
    const int4 ch = chunks[cid];
    const int64_t row = ch.x;
    constexpr int UN = 4;
    for (int h0 = 0; h0 < heads; h0 += NH) {
        float si[NH], m[NH], sm[NH];
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            si[k] = src[row * heads + h0 + k];
            m[k] = -INFINITY;
            sm[k] = 0.0f;
        }
        // the next batch's column indices are loaded behind this batch's
        // dst gathers
        int cn[UN];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
            const int i = ch.y + u * GL + lane;
            cn[u] = i < ch.z ? ci[i] : 0;
        }
        for (int i0 = ch.y; i0 < ch.z; i0 += GL * UN) {
            float x[UN][NH];
            bool ok[UN];
#pragma unroll
            for (int u = 0; u < UN; ++u) {
                ok[u] = i0 + u * GL + lane < ch.z;
                gat_dst<NH>(dst, heads, h0, cn[u], x[u]);
            }
            if (i0 + GL * UN < ch.z) {  // uniform per group
#pragma unroll
                for (int u = 0; u < UN; ++u) {
                    const int i = i0 + GL * UN + u * GL + lane;
                    cn[u] = i < ch.z ? ci[i] : 0;
                }
            }
#pragma unroll
            for (int k = 0; k < NH; ++k) {
                float bm = m[k];
#pragma unroll
                for (int u = 0; u < UN; ++u) {
                    x[u][k] = lrelu(si[k] + x[u][k], slope);
                    const float y = ok[u] ? x[u][k] : -INFINITY;
                    bm = (bm < y) ? y : bm;
                }
                // the running sum in units of the new max (an unchanged max
                // scales by exactly 1; the first batch's by exp(-inf) = 0)
                float acc = (bm == -INFINITY) ? 0.0f : sm[k] * expf(m[k] - bm);
#pragma unroll
                for (int u = 0; u < UN; ++u) {
                    const float p = expf(x[u][k] - bm);
                    acc = ok[u] ? acc + p : acc;
                }
                m[k] = bm;
                sm[k] = acc;
            }
        }
#pragma unroll
        for (int off = GL / 2; off >= 1; off >>= 1) {
#pragma unroll
            for (int k = 0; k < NH; ++k)
                softmax_merge(m[k], sm[k], __shfl_xor(m[k], off), __shfl_xor(sm[k], off));
        }
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            if (lane == k) {
                if (ch.w < 0) {
                    rmax[row * heads + h0 + k] = m[k];
                    rinv[row * heads + h0 + k] = (sm[k] > 0.0f) ? 1.0f / sm[k] : 0.0f;
                } else {
                    float* st = pstats + (static_cast<int64_t>(ch.w) * heads + h0 + k) * 2;
                    st[0] = m[k];
                    st[1] = sm[k];
                }
            }
        }
    }
}

// Exact statistics (the plan splits no row): one wave per row, heads in
// groups of NH.  The row's maximum score (order-independent, the max kept as
// (m < x) ? x : m), then the reference's sum of t_ij = exp_rn(e_ij - max) in
// nonzero order (layers.cpp:1076-1084): the lanes evaluate 64 entries' t at
// a time and the wave adds them one by one, in order, through readlane.
template <int NH>
__global__ __launch_bounds__(256) void gat_exact_stats_kernel(const int4* __restrict__ chunks,
                                                              int64_t n_chunks,
                                                              const int32_t* __restrict__ ci,
                                                              int heads,
                                                              const float* __restrict__ src,
                                                              const float* __restrict__ dst,
                                                              float slope,
                                                              float* __restrict__ rmax,
                                                              float* __restrict__ rinv) {
    const int lane = threadIdx.x & 63;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (cid >= n_chunks) return;  // uniform per wave
    const int4 ch = chunks[cid];
    const int64_t row = ch.x;
    for (int h0 = 0; h0 < heads; h0 += NH) {
        float si[NH], m[NH], sum[NH];
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            si[k] = src[row * heads + h0 + k];
            m[k] = -INFINITY;
            sum[k] = 0.0f;
        }
        for (int i = ch.y + lane; i < ch.z; i += 64) {
            float d[NH];
            gat_dst<NH>(dst, heads, h0, ci[i], d);
#pragma unroll
            for (int k = 0; k < NH; ++k) {
                const float x = lrelu(si[k] + d[k], slope);
                m[k] = (m[k] < x) ? x : m[k];
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
#pragma unroll
            for (int k = 0; k < NH; ++k) {
                const float o = __shfl_xor(m[k], off);
                m[k] = (m[k] < o) ? o : m[k];
            }
        }
        for (int i0 = ch.y; i0 < ch.z; i0 += 64) {
            const int i = i0 + lane;
            float t[NH];
            if (i < ch.z) {
                float d[NH];
                gat_dst<NH>(dst, heads, h0, ci[i], d);
#pragma unroll
                for (int k = 0; k < NH; ++k) t[k] = exp_rn(lrelu(si[k] + d[k], slope) - m[k]);
            } else {
#pragma unroll
                for (int k = 0; k < NH; ++k) t[k] = 0.0f;
            }
            const int cnt = ch.z - i0 < 64 ? ch.z - i0 : 64;
            for (int q = 0; q < cnt; ++q) {
#pragma unroll
                for (int k = 0; k < NH; ++k)
                    sum[k] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[k]), q));
            }
        }
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            if (lane == k) {
                rmax[row * heads + h0 + k] = m[k];
                rinv[row * heads + h0 + k] = (sum[k] > 0.0f) ? 1.0f / sum[k] : 0.0f;
            }
        }
    }
}

// Split rows: the chunks' (max, sum) pairs merged in chunk order, one
// thread per row and head.
__global__ __launch_bounds__(256) void gat_stats_merge_kernel(const int4* __restrict__ split,
                                                              int64_t n_split, int heads,
                                                              const float* __restrict__ pstats,
                                                              float* __restrict__ rmax,
                                                              float* __restrict__ rinv) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n_split * heads) return;
    const int4 sp = split[t / heads];
    const int h = static_cast<int>(t % heads);
    float m = -INFINITY, s = 0.0f;
    for (int c = 0; c < sp.z; ++c) {
        const float* st = pstats + (static_cast<int64_t>(sp.y + c) * heads + h) * 2;
        softmax_merge(m, s, st[0], st[1]);
    }
    rmax[static_cast<int64_t>(sp.x) * heads + h] = m;
    rinv[static_cast<int64_t>(sp.x) * heads + h] = (s > 0.0f) ? 1.0f / s : 0.0f;
}

// ---------------------------------------------------------------------------
// Blocked GAT passes with the softmax carried across the passes (fast
// precision): no statistics sweep.  Every (row, column group) keeps a
// running max m and a running sum s of exp(e - m) in state arrays
// [n x G] (G = the launch's column groups, grid.y), and the output row
// holds the unnormalised sum of exp(e_ij - m) Wh_j over the blocks so far.
// A pass raises m to the maximum of its entries' scores, rescaling the
// carried sum and output by exp(m_old - m_new) (the online softmax of
// gat_chunk_kernel, across blocks); the last pass multiplies by 1/s and
// applies bias and activations.  One lane group of LPR lanes (VEC 4 floats
// each) covers one column group of one chunk, inside one head.  The groups
// of a head compute the same m and s from the same entries in the same
// order; each keeps its own copy, so every state slot has a single owner
// per pass.  Rows split into several chunks leave per-chunk (m, s, sum)
// partials, merged with the state by gat_online_reduce_kernel.
// ---------------------------------------------------------------------------
struct GatPass {
    const float* src;  // [n x heads] a_l . Wh_i
    const float* dst;  // [n x heads] a_r . Wh_j
    // [heads x head_cols] a_r: the passes that hold a whole head per lane
    // group compute a_r . Wh_j from the gathered row instead of gathering dst
    const float* att_r;
    int tail_mask;     // those passes: the head's width is not a multiple of 4
    float* m_state;    // [n x G] running max per row and column group
    float* s_state;    // [n x G] running sum
    float* pstats;     // [partial slots x G x 2] (m, s) of split rows' chunks
    const float* bias;
    int heads;
    int head_cols;
    float slope;
    int act, post;
    int first, last;   // the pass's position among the blocks
    int vec_io;        // output rows 16-byte aligned: vector loads / stores
};

__device__ __forceinline__ void ld4_nt(const float* p, float (&x)[4]) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4 t = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
    x[0] = t.x;
    x[1] = t.y;
    x[2] = t.z;
    x[3] = t.w;
}

__device__ __forceinline__ void st4_nt(float* p, const float (&x)[4]) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    v4 t;
    t.x = x[0];
    t.y = x[1];
    t.z = x[2];
    t.w = x[3];
    __builtin_nontemporal_store(t, reinterpret_cast<v4*>(p));
}

// The output row's four floats at fo (those below f), vector or element-wise.
__device__ __forceinline__ void out_load(const float* row, int64_t fo, int64_t f, bool vec,
                                         float (&x)[4]) {
    if (vec) {
        ld4_nt(row + fo, x);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = fo + k < f ? row[fo + k] : 0.0f;
    }
}

__device__ __forceinline__ void out_store(float* row, int64_t fo, int64_t f, bool vec,
                                          const float (&x)[4]) {
    if (vec) {
        st4_nt(row + fo, x);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (fo + k < f) row[fo + k] = x[k];
    }
}

// The maximum over an aligned group of LPR (8 or 16) lanes with DPP moves,
// no LDS: max is exact, so the butterfly's order gives the same value as any.
template <int LPR>
__device__ __forceinline__ float group_max_dpp(float x) {
    static_assert(LPR == 8 || LPR == 16, "group width");
    float o;
    if constexpr (LPR == 16) {
        o = dpp_flip<8>(x);
        x = (x < o) ? o : x;
    }
    o = dpp_flip<4>(x);
    x = (x < o) ? o : x;
    o = dpp_flip<2>(x);
    x = (x < o) ? o : x;
    o = dpp_flip<1>(x);
    return (x < o) ? o : x;
}

// TMASK: the head's last lane holds fewer than four Wh columns (a_r . Wh_j
// masks the row padding).  OFF32: every gather's byte offset from B fits 32
// bits, and its column and the row pitch 24 (the host checks), so gathers
// take B as a scalar base and a 32-bit lane offset (one 24-bit multiply-add
// per gather instead of a 64-bit one).
template <int LPR, bool DIN, bool TMASK, bool OFF32>
__global__ __launch_bounds__(256, 4) void gat_online_chunk_kernel(
    const int4* __restrict__ chunks, int64_t n_chunks, const int32_t* __restrict__ ci,
    const uint16_t* __restrict__ ci16, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, float* __restrict__ partials, int64_t ldp, int64_t f,
    GatPass P) {
    constexpr int U = 16;                    // row gathers in flight per lane
    constexpr int CPL = U > LPR ? U / LPR : 1;
    constexpr int BE = LPR * CPL;            // entries per batch (== U)
    static_assert(BE == U, "one gather step per batch");
    constexpr int GPB = 256 / LPR;
    constexpr int TILE = LPR * 4;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t cid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (cid >= n_chunks) return;
    const int4 ch = chunks[cid];
    const int e = ch.z;
    // a middle pass leaves rows without entries in its block as they are
    if (!P.first && !P.last && ch.z == ch.y) return;
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    const int h = static_cast<int>(fbase / P.head_cols);
    const float si = P.src[static_cast<int64_t>(ch.x) * P.heads + h];
    const float* dh = P.dst + h;
    const int64_t so = static_cast<int64_t>(ch.x) * gridDim.y + blockIdx.y;  // state slot
    const int64_t fo = fbase + static_cast<int64_t>(l) * 4;
    const bool ok = fo < f;
    const int64_t fl = ok ? fo : fbase;  // lanes past f gather the tile's first vector
    float* crow = C + static_cast<int64_t>(ch.x) * ldc;
    // DIN (the group's columns are one whole head): a_r at the lane's
    // columns, 0 past the head; nv of the lane's four gathered floats are
    // Wh columns (the rest may be row padding, masked when tail_mask)
    float ar[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int nv = 0;
    if constexpr (DIN) {
        const int64_t hc = fo - static_cast<int64_t>(h) * P.head_cols;  // column in the head
        nv = ok ? static_cast<int>(P.head_cols - hc < 4 ? P.head_cols - hc : 4) : 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            ar[k] = k < nv ? P.att_r[static_cast<int64_t>(h) * P.head_cols + hc + k] : 0.0f;
    }

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, s = 0.0f;  // s: this lane's share of the running sum
    const bool unsplit = ch.w < 0;
    if (unsplit && !P.first) {
        m = P.m_state[so];
        if (l == 0) s = P.s_state[so];  // the carried sum, counted once in the group
        if (ok) out_load(crow, fo, f, P.vec_io, acc);
    }

    const char* bl = reinterpret_cast<const char*>(B + fl);
    const char* bs = reinterpret_cast<const char*>(B);
    const uint32_t loff = static_cast<uint32_t>(fl) * 4u;
    const uint32_t pitch = static_cast<uint32_t>(ldb) * 4u;
    const int stride = P.heads;
    int ncl[CPL];
    auto fetch = [&](int base) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int idx = base + l * CPL + j;
            ncl[j] = idx < e ? (ci16 ? static_cast<int>(ci16[idx]) : ci[idx]) : 0;
        }
    };
    fetch(ch.y);
    for (int base = ch.y; base < e; base += BE) {
        int cl[CPL];
        float d[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            cl[j] = ncl[j];
            // before the row gathers (DIN: from them, below)
            if constexpr (!DIN) d[j] = dh[static_cast<int64_t>(cl[j]) * stride];
        }
        const int cnt = e - base < BE ? e - base : BE;
        float bv[U][4];
        // entry u of the batch is slot u % CPL of lane u / CPL: compile-time
        // lanes, broadcast without LDS (group_bcast)
        static_for<0, U>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int col = group_bcast<LPR, u / CPL>(cl[u % CPL]);
            if constexpr (OFF32) {  // col and pitch below 2^24
                const uint32_t off = __umul24(static_cast<uint32_t>(col), pitch) + loff;
                ldv<4>(reinterpret_cast<const float*>(bs + off), bv[u]);
            } else {
                const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(col)) * pitch;
                ldv<4>(reinterpret_cast<const float*>(bl + off), bv[u]);
            }
        });
        fetch(base + BE);
        if constexpr (DIN) {
            // a_r . Wh_j of the batch's entries: the lane's four-column
            // share of each, summed over the group, entry l * CPL + j's
            // total landing in lane l (group_transpose_sum)
            float pd[U];
            static_for<0, U>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                float b1 = bv[u][1], b2 = bv[u][2], b3 = bv[u][3];
                if constexpr (TMASK) {
                    b1 = nv > 1 ? b1 : 0.0f;
                    b2 = nv > 2 ? b2 : 0.0f;
                    b3 = nv > 3 ? b3 : 0.0f;
                }
                float t = ar[0] * bv[u][0];
                t = __builtin_fmaf(ar[1], b1, t);
                t = __builtin_fmaf(ar[2], b2, t);
                pd[u] = __builtin_fmaf(ar[3], b3, t);
            });
            group_transpose_sum<LPR>(pd, l);
#pragma unroll
            for (int j = 0; j < CPL; ++j) d[j] = pd[j];
        }
        // the batch's scores, the group's maximum, the rescaled carry
        float ev[CPL];
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            ev[j] = lrelu(si + d[j], P.slope);
            if (base + l * CPL + j < e) bm = (bm < ev[j]) ? ev[j] : bm;
        }
        bm = group_max_dpp<LPR>(bm);
        if (m < bm) {  // uniform in the group
            const float fct = expf(m - bm);  // 0 when nothing was carried (m = -inf)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] *= fct;
            s *= fct;
            m = bm;
        }
        float wl[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            wl[j] = base + l * CPL + j < e ? expf(ev[j] - m) : 0.0f;
            s += wl[j];
        }
        if (cnt == BE) {  // a full batch: every slot is an entry (no selects)
            static_for<0, U>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                const float w = group_bcast<LPR, u / CPL>(wl[u % CPL]);
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(w, bv[u][k], acc[k]);
            });
        } else {
            static_for<0, U>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                const float w = group_bcast<LPR, u / CPL>(wl[u % CPL]);
                const bool valid = u < cnt;  // a select, not a branch
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float nx = __builtin_fmaf(w, bv[u][k], acc[k]);
                    acc[k] = valid ? nx : acc[k];
                }
            });
        }
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, LPR);

    if (!unsplit) {
        if (ok) stv<4>(partials + static_cast<int64_t>(ch.w) * ldp + fo, acc);
        if (l == 0) {
            float* st = P.pstats + (static_cast<int64_t>(ch.w) * gridDim.y + blockIdx.y) * 2;
            st[0] = m;
            st[1] = s;
        }
        return;
    }
    if (P.last) {
        const float inv = s > 0.0f ? 1.0f / s : 0.0f;
        float x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            x[k] = finish_val(acc[k] * inv, P.bias, fo + k < f ? fo + k : fo, P.act, P.post);
        if (ok) out_store(crow, fo, f, P.vec_io, x);
        return;
    }
    if (ok) out_store(crow, fo, f, P.vec_io, acc);
    if (l == 0) {
        P.m_state[so] = m;
        P.s_state[so] = s;
    }
}

// Split rows of a pass: the state carried from the earlier passes and the
// chunks' (m_c, s_c, sum_c) merged into M = max, S = sum s exp(m - M), out =
// sum sum_c exp(m_c - M); the last pass normalises and applies the epilogue.
template <int LPR>
__global__ __launch_bounds__(256) void gat_online_reduce_kernel(
    const int4* __restrict__ split, int64_t n_split, const float* __restrict__ partials,
    int64_t ldp, float* __restrict__ C, int64_t ldc, int64_t f, GatPass P) {
    constexpr int GPB = 256 / LPR;
    constexpr int TILE = LPR * 4;
    const int g = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int64_t sid = static_cast<int64_t>(blockIdx.x) * GPB + g;
    if (sid >= n_split) return;
    const int4 sp = split[sid];
    const int64_t fbase = static_cast<int64_t>(blockIdx.y) * TILE;
    const int64_t so = static_cast<int64_t>(sp.x) * gridDim.y + blockIdx.y;  // state slot
    const int64_t fo = fbase + static_cast<int64_t>(l) * 4;
    const bool ok = fo < f;
    float* crow = C + static_cast<int64_t>(sp.x) * ldc;
    float mp = -INFINITY, sprev = 0.0f, prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (!P.first) {
        mp = P.m_state[so];
        sprev = P.s_state[so];
        if (ok) out_load(crow, fo, f, P.vec_io, prev);
    }
    float M = mp;
    for (int c = 0; c < sp.z; ++c) {
        const float mc = P.pstats[(static_cast<int64_t>(sp.y + c) * gridDim.y + blockIdx.y) * 2];
        M = (M < mc) ? mc : M;
    }
    const float fp = expf(mp - M);  // 0 when nothing was carried
    float S = sprev * fp, acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = prev[k] * fp;
    for (int c = 0; c < sp.z; ++c) {
        const float* st =
            P.pstats + (static_cast<int64_t>(sp.y + c) * gridDim.y + blockIdx.y) * 2;
        const float fc = expf(st[0] - M);
        S += st[1] * fc;
        if (ok) {
            float t[4];
            ldv<4>(partials + static_cast<int64_t>(sp.y + c) * ldp + fo, t);
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(t[k], fc, acc[k]);
        }
    }
    if (P.last) {
        const float inv = S > 0.0f ? 1.0f / S : 0.0f;
        float x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            x[k] = finish_val(acc[k] * inv, P.bias, fo + k < f ? fo + k : fo, P.act, P.post);
        if (ok) out_store(crow, fo, f, P.vec_io, x);
        return;
    }
    if (ok) out_store(crow, fo, f, P.vec_io, acc);
    if (l == 0) {
        P.m_state[so] = M;
        P.s_state[so] = S;
    }
}

template <int LPR, bool DIN>
void gat_online_passes(const BlockedCSR& bk, int64_t f, const float* wh, int64_t ldwh,
                       float* out, int64_t ldo, const GatPass& base, int64_t max_partials,
                       hipStream_t s) {
    constexpr int GPB = 256 / LPR;
    const int64_t ldp = round_up(f, 4);
    const unsigned ytiles = static_cast<unsigned>(ceil_div(f, LPR * 4));
    // gather offsets from a block's first row: (column within the block) x
    // row pitch + column offset, all in 32 bits when they fit
    const int64_t rows_in = bk.idx16 ? bk.rows_per_block : bk.n;
    const bool off32 = rows_in * ldwh * 4 + ldwh * 4 < (int64_t(1) << 32) &&
                       rows_in < (int64_t(1) << 24) && ldwh * 4 < (int64_t(1) << 24);
    for (int64_t blk = 0; blk < bk.n_blocks; ++blk) {
        const tg_spmm_plan_s& p = *bk.plans[blk];
        require(p.n_partials <= max_partials, "GATLayer: block plan has more partial slots");
        GatPass P = base;
        P.first = blk == 0;
        P.last = blk + 1 == bk.n_blocks;
        if (p.n_chunks > 0) {
            // 16-bit indices count from the block's first source row
            const int64_t r0 = bk.idx16 ? blk * bk.rows_per_block : 0;
            GatPass Q = P;
            Q.dst = P.dst + r0 * P.heads;
            dim3 grid(static_cast<unsigned>(ceil_div(p.n_chunks, GPB)), ytiles);
            const int32_t* ci = bk.idx16 ? nullptr : bk.bci.as<int32_t>();
            const uint16_t* ci16 = bk.idx16 ? bk.bci.as<uint16_t>() : nullptr;
            const float* bb = wh + r0 * ldwh;
            float* pp = p.partials.as<float>();
#define TG_GAT_ONLINE(TM_, O32_)                                                         \
    gat_online_chunk_kernel<LPR, DIN, TM_, O32_><<<grid, 256, 0, s>>>(                  \
        p.chunks.as<int4>(), p.n_chunks, ci, ci16, bb, ldwh, out, ldo, pp, ldp, f, Q)
            if (Q.tail_mask) {
                if (off32) TG_GAT_ONLINE(true, true); else TG_GAT_ONLINE(true, false);
            } else {
                if (off32) TG_GAT_ONLINE(false, true); else TG_GAT_ONLINE(false, false);
            }
#undef TG_GAT_ONLINE
            TG_LAUNCH_CHECK();
        }
        if (p.n_split > 0) {
            dim3 grid(static_cast<unsigned>(ceil_div(p.n_split, GPB)), ytiles);
            gat_online_reduce_kernel<LPR><<<grid, 256, 0, s>>>(
                p.split.as<int4>(), p.n_split, p.partials.as<float>(), ldp, out, ldo, f, P);
            TG_LAUNCH_CHECK();
        }
    }
}

size_t gat_ws_partials(int64_t n_partials, int64_t n, int64_t heads, int64_t f, int concat) {
    Carver c(nullptr, 0);
    c.take<float>(std::max<int64_t>(n_partials, 1) * gat_stat_slots(heads, f) * 2);
    if (!concat && heads > 1) c.take<float>(n * heads * f);
    return c.bytes();
}

}  // namespace

void gat_scores(int64_t n, int64_t heads, int64_t f, const float* wh, int64_t ldwh,
                const float* al, const float* ar, float* src, float* dst, hipStream_t s) {
    require(n >= 0 && heads >= 1 && f >= 1, "GATLayer: bad sizes");
    require(ldwh >= heads * f, "GATLayer: Wh leading dimension too small");
    require(heads * f < (int64_t(1) << 31), "GATLayer: heads * f too large");
    if (n == 0) return;
    require(wh && al && ar && src && dst, "GATLayer: null pointer");
    const bool al16 = reinterpret_cast<uintptr_t>(wh) % 16 == 0;
    const int64_t f4x4 = round_up(f, 4);
    const bool segs = f % 4 == 0 || (heads == 1 && ldwh >= f4x4);  // whole vectors per segment
    if (f <= 64 && segs && ldwh % 4 == 0 && al16 && heads <= 16) {
        const size_t lds = static_cast<size_t>(kScorePairs + 2 * heads) * (f4x4 + 1) * sizeof(float);
        gat_scores_lds_kernel<<<static_cast<unsigned>(ceil_div(n * heads, kScorePairs)),
                                kScorePairs, lds, s>>>(n, static_cast<int>(heads),
                                                       static_cast<int>(f), wh, ldwh, al, ar, src,
                                                       dst);
    } else {
        gat_scores_kernel<<<static_cast<unsigned>(ceil_div(n * heads, 256)), 256, 0, s>>>(
            n, static_cast<int>(heads), static_cast<int>(f), wh, ldwh, al, ar, src, dst);
    }
    TG_LAUNCH_CHECK();
}

size_t gat_workspace(const tg_spmm_plan_s& p, int64_t n, int64_t heads, int64_t f, int concat) {
    return gat_ws_partials(p.n_partials, n, heads, f, concat);
}

int64_t blocked_max_partials(const BlockedCSR& bk) {
    int64_t m = 0;
    for (const auto& p : bk.plans) m = std::max(m, p->n_partials);
    return m;
}

size_t gat_workspace_blocked(const BlockedCSR& bk, int64_t n, int64_t heads, int64_t f,
                             int concat) {
    return gat_ws_partials(blocked_max_partials(bk), n, heads, f, concat);
}

void gat_aggregate(const tg_spmm_plan_s& p, int64_t n, int64_t heads, int64_t f,
                   const int32_t* ci, const float* wh, int64_t ldwh, const float* src,
                   const float* dst, float slope, const float* bias, int act, int post,
                   int concat, float* out, int64_t ldo, void* work, size_t work_bytes,
                   hipStream_t s, bool exact) {
    require(n == p.m, "GATLayer::forward: plan rows differ from n");
    require(heads >= 1 && f >= 1, "GATLayer: bad sizes");
    require(act == TG_ACT_NONE || act == TG_ACT_RELU, "GATLayer: unknown activation");
    require(post >= TG_POST_NONE && post <= TG_POST_ELU, "GATLayer: unknown post activation");
    const int64_t ftot = heads * f;
    require(ldwh >= ftot, "GATLayer: Wh leading dimension too small");
    const bool avg = !concat && heads > 1;
    require(ldo >= (avg ? f : ftot), "GATLayer: output leading dimension too small");
    if (n == 0) return;
    if (p.n_split > 0)
        require(ftot <= p.max_f, "GATLayer: heads * f exceeds the plan's max_f");
    DeviceBuffer own;
    if (work == nullptr) {
        own.resize(gat_ws_partials(p.n_partials, n, heads, f, concat));
        work = own.get();
        work_bytes = own.size();
    }
    Carver c(work, work_bytes);
    float* pstats = c.take<float>(std::max<int64_t>(p.n_partials, 1) * heads * 2);
    float* tmp = avg ? c.take<float>(n * ftot) : nullptr;

    GatArgs a{};
    a.chunks = p.chunks.as<int4>();
    a.n_chunks = p.n_chunks;
    a.split = p.split.as<int4>();
    a.n_split = p.n_split;
    a.ci = ci;
    a.wh = wh;
    a.ldwh = ldwh;
    a.src = src;
    a.dst = dst;
    a.heads = static_cast<int>(heads);
    a.f = static_cast<int>(f);
    a.ftot = ftot;
    a.slope = slope;
    a.out = avg ? tmp : out;
    a.ldo = avg ? ftot : ldo;
    a.partials = p.partials.as<float>();
    a.pstats = pstats;
    a.bias = bias;
    a.act = act;
    a.post = avg ? TG_POST_NONE : post;
    a.exact = exact ? 1 : 0;
    // Loads: the widest access the rows of Wh allow, never straddling two
    // heads (the width divides f, or there is one head); stores and bias
    // loads are vectors only when aligned as well.
    int vec = pick_load_vec(ftot, ldwh, wh);
    while (vec > 1 && heads > 1 && f % vec != 0) vec /= 2;
    a.ldp = round_up(ftot, vec);
    a.vec_io = pick_vec(ftot, {a.ldo}, {a.out, bias}) >= vec;
    const LaneLayout L = choose_layout(ftot, vec);
    if (vec == 4)
        dispatch_gat<4>(p, L, a, s);
    else if (vec == 2)
        dispatch_gat<2>(p, L, a, s);
    else
        dispatch_gat<1>(p, L, a, s);
    if (avg) {
        gat_average_kernel<<<static_cast<unsigned>(ceil_div(n * f, 256)), 256, 0, s>>>(
            tmp, n, static_cast<int>(heads), static_cast<int>(f), out, ldo, post, exact ? 1 : 0);
        TG_LAUNCH_CHECK();
    }
    if (own.get()) TG_HIP(hipStreamSynchronize(s));
}

bool gat_blocked_ok(int64_t heads, int64_t f, int concat) {
    if (!concat && heads > 1) return false;      // head average: unblocked kernel
    return heads == 1 || f % 32 == 0;            // 32-column tiles inside one head
}

void gat_aggregate_blocked(const BlockedCSR& bk, const tg_spmm_plan_s* plan, int64_t n,
                           int64_t heads, int64_t f, const int32_t* ci, const float* wh,
                           int64_t ldwh, const float* src, const float* dst, float slope,
                           const float* bias, int act, int post, float* out, int64_t ldo,
                           float* rmax, float* rinv, void* work, size_t work_bytes,
                           hipStream_t s, bool exact, const float* ar) {
    require(bk.n == n && (plan == nullptr || plan->m == n),
            "GATLayer: blocked structure or plan rows differ from n");
    require(gat_blocked_ok(heads, f, 1), "GATLayer: layout not supported blocked");
    require(heads * f < (int64_t(1) << 31), "GATLayer: heads * f too large");
    if (n == 0) return;
    // fast precision, each head inside one lane group's columns and Wh rows
    // 16-byte aligned: the softmax rides along the passes (no statistics
    // sweep); the lane-group width is the one run_aggregate_blocked picks
    const int64_t ftot = heads * f;
    const bool wide = bk.group_cols == 64 && ftot > 32 && (f >= ftot || f % 64 == 0);
    const int gc = wide ? 64 : 32;
    const bool online = !exact && (heads == 1 || f % gc == 0) && ldwh % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(wh) % 16 == 0;
    if (online) {
        // state per (row, column group): G <= gat_stat_slots(heads, f)
        const int64_t groups = ceil_div(ftot, gc);
        Carver cw(work, work_bytes);
        GatPass P{};
        P.src = src;
        P.dst = dst;
        P.att_r = ar;
        P.tail_mask = f % 4 != 0 ? 1 : 0;
        P.m_state = rmax;
        P.s_state = rinv;
        P.pstats = cw.take<float>(std::max<int64_t>(blocked_max_partials(bk), 1) * groups * 2);
        P.bias = bias;
        P.heads = static_cast<int>(heads);
        P.head_cols = static_cast<int>(f);
        P.slope = slope;
        P.act = act;
        P.post = post;
        P.vec_io = ftot % 4 == 0 && ldo % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                   (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 16 == 0);
        // partial slots: the block plans' (work holds gat_workspace_blocked)
        const int64_t maxp = std::max<int64_t>(blocked_max_partials(bk), 1);
        // a whole head per lane group: a_r . Wh_j from the gathered rows (a
        // gather of dst per entry cost 2 ms of the config-E GAT forward's 11.8)
        const bool din = ar != nullptr && (heads == 1 ? f <= gc : f == gc);
        if (gc == 64) {
            if (din)
                gat_online_passes<16, true>(bk, ftot, wh, ldwh, out, ldo, P, maxp, s);
            else
                gat_online_passes<16, false>(bk, ftot, wh, ldwh, out, ldo, P, maxp, s);
        } else {
            if (din)
                gat_online_passes<8, true>(bk, ftot, wh, ldwh, out, ldo, P, maxp, s);
            else
                gat_online_passes<8, false>(bk, ftot, wh, ldwh, out, ldo, P, maxp, s);
        }
        return;
    }
    require(plan != nullptr, "GATLayer: the statistics need the unblocked plan");
    const tg_spmm_plan_s& p = *plan;
    const bool vec4 = heads % 4 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    const unsigned grid = static_cast<unsigned>(ceil_div(p.n_chunks, 4));
    if (exact) {
        // the reference's operation order: the plan splits no row, the
        // blocked rows are in block order, each pass continues the chains
        require(p.n_split == 0 && bk.in_order,
                "GATLayer: the exact blocked path needs unsplit, in-order rows");
        if (p.n_chunks > 0) {
            if (vec4)
                gat_exact_stats_kernel<4><<<grid, 256, 0, s>>>(p.chunks.as<int4>(), p.n_chunks,
                                                               ci, static_cast<int>(heads), src,
                                                               dst, slope, rmax, rinv);
            else
                gat_exact_stats_kernel<1><<<grid, 256, 0, s>>>(p.chunks.as<int4>(), p.n_chunks,
                                                               ci, static_cast<int>(heads), src,
                                                               dst, slope, rmax, rinv);
            TG_LAUNCH_CHECK();
        }
    } else {
        // per-chunk (max, sum) pairs of split rows: the unblocked path's pstats
        Carver cw(work, work_bytes);
        float* pstats = cw.take<float>(std::max<int64_t>(p.n_partials, 1) * heads * 2);
        if (p.n_chunks > 0) {
            // two chunks per wave (config-E GAT forward: 64 lanes per chunk
            // 14.24 ms, 32 lanes 14.14 ms, 16 lanes 14.17 ms)
            constexpr int kGL = 32;
            const unsigned sgrid = static_cast<unsigned>(ceil_div(p.n_chunks, 256 / kGL));
            if (vec4)
                gat_stats_kernel<4, kGL><<<sgrid, 256, 0, s>>>(p.chunks.as<int4>(), p.n_chunks, ci,
                                                              static_cast<int>(heads), src, dst,
                                                              slope, rmax, rinv, pstats);
            else
                gat_stats_kernel<1, kGL><<<sgrid, 256, 0, s>>>(p.chunks.as<int4>(), p.n_chunks, ci,
                                                              static_cast<int>(heads), src, dst,
                                                              slope, rmax, rinv, pstats);
            TG_LAUNCH_CHECK();
        }
        if (p.n_split > 0) {
            gat_stats_merge_kernel<<<static_cast<unsigned>(ceil_div(p.n_split * heads, 256)), 256,
                                     0, s>>>(p.split.as<int4>(), p.n_split,
                                             static_cast<int>(heads), pstats, rmax, rinv);
            TG_LAUNCH_CHECK();
        }
    }
    // the passes compute alpha_ij per entry and head from the scores and
    // the row statistics: the nnz x heads attention matrix is never stored
    AggEpilogue epi;
    epi.bias = bias;
    epi.act = act;
    epi.post = post;
    epi.exact_exp = exact ? 1 : 0;
    epi.w_head_cols = static_cast<int>(f);
    epi.att_src = src;
    epi.att_dst = dst;
    epi.att_max = rmax;
    epi.att_rinv = rinv;
    epi.att_heads = static_cast<int>(heads);
    epi.att_slope = slope;
    run_aggregate_blocked(bk, heads * f, wh, ldwh, out, ldo, epi, s);
}

}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_gat_scores(int64_t n, int64_t heads, int64_t f, const float* wh, int64_t ldwh,
                  const float* att_l, const float* att_r, float* src, float* dst,
                  tg_stream_t stream) {
    return guard([&] {
        tg::gat_scores(n, heads, f, wh, ldwh, att_l, att_r, src, dst,
                       static_cast<hipStream_t>(stream));
    });
}

size_t tg_gat_workspace_size(tg_spmm_plan_t plan, int64_t n, int64_t heads, int64_t f,
                             int concat) {
    if (plan == nullptr || heads < 1 || f < 1 || n < 0) return 0;
    return tg::gat_workspace(*plan, n, heads, f, concat);
}

int tg_gat_aggregate(tg_spmm_plan_t plan, int64_t n, int64_t heads, int64_t f,
                     const int32_t* row_ptr, const int32_t* col_ind, const float* wh,
                     int64_t ldwh, const float* src, const float* dst, float slope,
                     const float* bias, int act, int post, int concat, float* out, int64_t ldo,
                     void* workspace, size_t workspace_bytes, tg_stream_t stream) {
    return guard([&] {
        require(plan != nullptr, "GATLayer::forward: plan is null");
        require(row_ptr == plan->row_ptr, "GATLayer::forward: row_ptr differs from the plan's");
        tg::gat_aggregate(*plan, n, heads, f, col_ind, wh, ldwh, src, dst, slope, bias, act, post,
                          concat, out, ldo, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream), false);
    });
}

}  // extern "C"
