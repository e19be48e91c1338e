/*
 * tg_oracle.c -- CPU restatement of TinyGNN's sparse-inference path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see
 * tg_oracle.h.  Compiled by oracle/Makefile with
 *   gcc -O3 -mavx2 -mfma -funroll-loops -fopenmp -ffp-contract=off
 * so that exactly the fmaf() calls below are fused and nothing else.
 *
 * Citations are reference file:line (src/ops.cpp, src/layers.cpp,
 * src/graph_loader.cpp).
 */
#include "tg_oracle.h"

#include <errno.h>
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

static __thread char g_err[8192];

const char* or_last_error(void) { return g_err; }

void or_set_num_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}

int or_get_num_threads(void) { return omp_get_max_threads(); }

/* ------------------------------------------------------------------------
 * graph_loader.cpp:211-281  edge_list_to_csr
 *   1. validate endpoints (throws invalid_argument)      :227-242
 *   2. out-degree count per src                          :244-248
 *   3. exclusive prefix sum -> row_ptr                   :250-254
 *   4. scatter dst in input order with per-row cursor    :256-264
 *   5. std::sort each row (duplicates kept)              :266-271
 *   6. values all 1.0f                                   :273-274
 * The per-row sort is done here with qsort in parallel over rows: the
 * sorted multiset of a row is unique, so any correct sort yields the same
 * bytes as std::sort.
 * ------------------------------------------------------------------------ */
static int cmp_i32(const void* a, const void* b) {
    const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

static void sort_small_i32(int32_t* p, int64_t n) {
    for (int64_t i = 1; i < n; ++i) {
        int32_t v = p[i];
        int64_t j = i - 1;
        while (j >= 0 && p[j] > v) { p[j + 1] = p[j]; --j; }
        p[j + 1] = v;
    }
}

int or_edge_list_to_csr(int64_t n_nodes, int64_t n_edges,
                        const int32_t* src, const int32_t* dst,
                        int32_t* row_ptr, int32_t* col_ind, float* val) {
    if (n_nodes == 0) {
        if (n_edges != 0) {
            snprintf(g_err, sizeof g_err,
                     "GraphLoader::edge_list_to_csr: num_nodes is 0 but "
                     "edges is non-empty");
            return 1;
        }
        row_ptr[0] = 0;
        return 0;
    }
    for (int64_t i = 0; i < n_edges; ++i) {
        if (src[i] < 0 || (int64_t)src[i] >= n_nodes) {
            snprintf(g_err, sizeof g_err,
                     "GraphLoader::edge_list_to_csr: edge[%lld].src = %d "
                     "out of range [0, %lld)", (long long)i, src[i],
                     (long long)n_nodes);
            return 1;
        }
        if (dst[i] < 0 || (int64_t)dst[i] >= n_nodes) {
            snprintf(g_err, sizeof g_err,
                     "GraphLoader::edge_list_to_csr: edge[%lld].dst = %d "
                     "out of range [0, %lld)", (long long)i, dst[i],
                     (long long)n_nodes);
            return 1;
        }
    }
    int32_t* cursor = (int32_t*)calloc((size_t)n_nodes, sizeof(int32_t));
    for (int64_t i = 0; i < n_edges; ++i) cursor[src[i]]++;
    row_ptr[0] = 0;
    for (int64_t i = 0; i < n_nodes; ++i) row_ptr[i + 1] = row_ptr[i] + cursor[i];
    memset(cursor, 0, (size_t)n_nodes * sizeof(int32_t));
    for (int64_t i = 0; i < n_edges; ++i) {
        const int32_t s = src[i];
        col_ind[row_ptr[s] + cursor[s]] = dst[i];
        cursor[s]++;
    }
    free(cursor);
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t r = 0; r < n_nodes; ++r) {
        const int64_t len = row_ptr[r + 1] - row_ptr[r];
        if (len <= 32) sort_small_i32(col_ind + row_ptr[r], len);
        else qsort(col_ind + row_ptr[r], (size_t)len, sizeof(int32_t), cmp_i32);
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_edges; ++i) val[i] = 1.0f;
    return 0;
}

/* ------------------------------------------------------------------------
 * layers.cpp:71-144  add_self_loops
 *   pass 1 (:83-91): has_diag[i] = any col == i; extra = #rows without one
 *   pass 2 (:102-137): copy row; before the first col > i insert (i, 1.0f)
 *   when the row has no diagonal; every col == i entry becomes v + 1.0f;
 *   if still not written, append (i, 1.0f) at the row end.
 * ------------------------------------------------------------------------ */
static int row_has_diag(int64_t i, const int32_t* rp, const int32_t* ci) {
    for (int32_t nz = rp[i]; nz < rp[i + 1]; ++nz)
        if (ci[nz] == (int32_t)i) return 1;
    return 0;
}

int64_t or_add_self_loops_nnz(int64_t n, const int32_t* rp, const int32_t* ci) {
    int64_t extra = 0;
    for (int64_t i = 0; i < n; ++i)
        if (!row_has_diag(i, rp, ci)) ++extra;
    return (int64_t)rp[n] + extra;
}

void or_add_self_loops(int64_t n, const int32_t* rp, const int32_t* ci,
                       const float* v, int32_t* rp_out, int32_t* ci_out,
                       float* v_out) {
    int64_t pos = 0;
    for (int64_t i = 0; i < n; ++i) {
        rp_out[i] = (int32_t)pos;
        const int has_diag = row_has_diag(i, rp, ci);
        int diag_written = 0;
        for (int32_t nz = rp[i]; nz < rp[i + 1]; ++nz) {
            const int32_t col = ci[nz];
            if (!diag_written && !has_diag && col > (int32_t)i) {
                ci_out[pos] = (int32_t)i;
                v_out[pos] = 1.0f;
                ++pos;
                diag_written = 1;
            }
            if (col == (int32_t)i) {
                ci_out[pos] = col;
                v_out[pos] = v[nz] + 1.0f;
                ++pos;
                diag_written = 1;
            } else {
                ci_out[pos] = col;
                v_out[pos] = v[nz];
                ++pos;
            }
        }
        if (!diag_written) {
            ci_out[pos] = (int32_t)i;
            v_out[pos] = 1.0f;
            ++pos;
        }
    }
    rp_out[n] = (int32_t)pos;
}

/* ------------------------------------------------------------------------
 * layers.cpp:158-208  gcn_norm
 *   A~ = add_self_loops(A)                                  :162
 *   deg[i] = sequential fp32 sum of row values of A~         :170-178
 *   dis[i] = deg > 0 ? 1.0f / sqrtf(deg) : 0                 :181-187
 *   v'[nz] = (v[nz] * dis_i) * dis_j                         :190-198
 * ------------------------------------------------------------------------ */
void or_gcn_norm(int64_t n, const int32_t* rp, const int32_t* ci,
                 const float* v, int32_t* rp_out, int32_t* ci_out,
                 float* v_out, float* deg_out, float* dis_out) {
    const int64_t nnz_sl = or_add_self_loops_nnz(n, rp, ci);
    float* v_sl = (float*)malloc((size_t)(nnz_sl > 0 ? nnz_sl : 1) * sizeof(float));
    or_add_self_loops(n, rp, ci, v, rp_out, ci_out, v_sl);
    float* deg = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    float* dis = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float d = 0.0f;
        for (int32_t nz = rp_out[i]; nz < rp_out[i + 1]; ++nz) d += v_sl[nz];
        deg[i] = d;
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        dis[i] = (deg[i] > 0.0f) ? (1.0f / sqrtf(deg[i])) : 0.0f;
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < n; ++i) {
        const float dis_i = dis[i];
        for (int32_t nz = rp_out[i]; nz < rp_out[i + 1]; ++nz)
            v_out[nz] = v_sl[nz] * dis_i * dis[ci_out[nz]];
    }
    if (deg_out) memcpy(deg_out, deg, (size_t)n * sizeof(float));
    if (dis_out) memcpy(dis_out, dis, (size_t)n * sizeof(float));
    free(deg);
    free(dis);
    free(v_sl);
}

/* ------------------------------------------------------------------------
 * ops.cpp:198-297  spmm.  C starts at 0 (:231); per row, nonzeros in
 * order, C[i,j] = fma(val, B[col,j], C[i,j]) for every j (the AVX2 lanes of
 * :266-284 and the contracted scalar tail :285-287 are the same fma).
 * ------------------------------------------------------------------------ */
void or_spmm(int64_t m, int64_t f, const int32_t* rp, const int32_t* ci,
             const float* av, const float* b, float* c) {
    memset(c, 0, (size_t)(m * f) * sizeof(float));
    if (m == 0 || f == 0 || rp[m] == 0) return;
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < m; ++i) {
        float* crow = c + i * f;
        for (int32_t nz = rp[i]; nz < rp[i + 1]; ++nz) {
            const float a = av[nz];
            const float* brow = b + (int64_t)ci[nz] * f;
            for (int64_t j = 0; j < f; ++j) crow[j] = fmaf(a, brow[j], crow[j]);
        }
    }
}

/* ------------------------------------------------------------------------
 * Checker, not a restatement: the exact-in-double product of selected rows,
 * exact[r] = sum val * B[col] and absum[r] = sum |val * B[col]| over row
 * rows[r]'s nonzeros, in float64.  Each term is exact in double (a product
 * of two floats), so |fl32 sum - exact| <= k 2^-24 absum (+ the float64
 * rounding, far smaller) bounds any float32 summation order of k roundings:
 * the bound that regrouped (split-row) sums are held to.
 * ------------------------------------------------------------------------ */
void or_spmm_rows_f64(int64_t n_sel, const int32_t* rows, int64_t f, const int32_t* rp,
                      const int32_t* ci, const float* av, const float* b, double* exact,
                      double* absum) {
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < n_sel; ++r) {
        const int64_t i = rows[r];
        double* e = exact + r * f;
        double* s = absum + r * f;
        for (int64_t j = 0; j < f; ++j) e[j] = s[j] = 0.0;
        for (int32_t nz = rp[i]; nz < rp[i + 1]; ++nz) {
            const double a = av[nz];
            const float* brow = b + (int64_t)ci[nz] * f;
            for (int64_t j = 0; j < f; ++j) {
                const double t = a * (double)brow[j];
                e[j] += t;
                s[j] += fabs(t);
            }
        }
    }
}

/* ------------------------------------------------------------------------
 * ops.cpp:70-162  matmul, (i,k,j) order, C[i,j] = fma(A[i,k], B[k,j], C)
 * with k ascending from 0 and C starting at 0 (:106, :120-159).
 * ------------------------------------------------------------------------ */
void or_matmul(int64_t m, int64_t k, int64_t n, const float* a,
               const float* b, float* c) {
    memset(c, 0, (size_t)(m * n) * sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        float* ci = c + i * n;
        for (int64_t kk = 0; kk < k; ++kk) {
            const float aik = a[i * k + kk];
            const float* bk = b + kk * n;
            for (int64_t j = 0; j < n; ++j) ci[j] = fmaf(aik, bk[j], ci[j]);
        }
    }
}

/* ops.cpp:328-338: d = std::max(0.0f, d)  ==  (0.0f < d) ? d : 0.0f */
void or_relu(int64_t n, float* x) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) x[i] = (0.0f < x[i]) ? x[i] : 0.0f;
}

/* ops.cpp:355-365 */
void or_leaky_relu(int64_t n, float* x, float alpha) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] >= 0.0f ? x[i] : alpha * x[i];
}

/* ops.cpp:380-392 */
void or_elu(int64_t n, float* x, float alpha) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        if (x[i] < 0.0f) x[i] = alpha * (expf(x[i]) - 1.0f);
}

/* ops.cpp:411-426 */
void or_sigmoid(int64_t n, float* x) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        if (x[i] >= 0.0f) {
            x[i] = 1.0f / (1.0f + expf(-x[i]));
        } else {
            const float ex = expf(x[i]);
            x[i] = ex / (1.0f + ex);
        }
    }
}

/* ops.cpp:441-451 */
void or_tanh(int64_t n, float* x) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) x[i] = tanhf(x[i]);
}

/* ops.cpp:469-484 (tanh approximation).  C++ evaluation order kept:
 * x + COEFF*x*x*x is x + ((COEFF*x)*x)*x, whose last product GCC contracts
 * into fma((COEFF*x)*x, x, x); the outer product is (0.5f*x)*(1+tanh). */
void or_gelu(int64_t n, float* x) {
    const float k0 = 0.7978845608f, k1 = 0.044715f;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        const float inner = k0 * fmaf(k1 * v * v, v, v);
        x[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* ops.cpp:506-546 */
void or_softmax(int64_t m, int64_t n, float* x) {
    #pragma omp parallel for schedule(dynamic)
    for (int64_t i = 0; i < m; ++i) {
        float* row = x + i * n;
        float mx = row[0];
        for (int64_t j = 1; j < n; ++j) if (row[j] > mx) mx = row[j];
        float s = 0.0f;
        for (int64_t j = 0; j < n; ++j) { row[j] = expf(row[j] - mx); s += row[j]; }
        const float inv = 1.0f / s;
        for (int64_t j = 0; j < n; ++j) row[j] *= inv;
    }
}

/* ops.cpp:565-606 */
void or_log_softmax(int64_t m, int64_t n, float* x) {
    #pragma omp parallel for schedule(dynamic)
    for (int64_t i = 0; i < m; ++i) {
        float* row = x + i * n;
        float mx = row[0];
        for (int64_t j = 1; j < n; ++j) if (row[j] > mx) mx = row[j];
        float s = 0.0f;
        for (int64_t j = 0; j < n; ++j) s += expf(row[j] - mx);
        const float lse = mx + logf(s);
        for (int64_t j = 0; j < n; ++j) row[j] -= lse;
    }
}

/* ops.cpp:622-661 */
void or_add_bias(int64_t m, int64_t n, float* x, const float* bias) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) x[i * n + j] += bias[j];
}

/* layers.cpp:768-822  edge_softmax.  Empty rows untouched (their range is
 * empty); max, then exp and sequential sum, then multiply by 1/sum. */
void or_edge_softmax(int64_t n, const int32_t* rp, const float* v,
                     float* v_out) {
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < n; ++i) {
        const int32_t b = rp[i], e = rp[i + 1];
        if (b == e) continue;
        float mx = v[b];
        for (int32_t nz = b + 1; nz < e; ++nz) mx = (mx < v[nz]) ? v[nz] : mx;
        float s = 0.0f;
        for (int32_t nz = b; nz < e; ++nz) {
            const float t = expf(v[nz] - mx);
            v_out[nz] = t;
            s += t;
        }
        if (s > 0.0f) {
            const float inv = 1.0f / s;
            for (int32_t nz = b; nz < e; ++nz) v_out[nz] *= inv;
        }
    }
}

/* layers.cpp:359-435  sage_max_aggregate: -inf start for nonempty rows,
 * element-wise std::max(acc, h) (acc < h ? h : acc), empty rows stay 0. */
void or_sage_max_aggregate(int64_t n, int64_t f, const int32_t* rp,
                           const int32_t* ci, const float* h, float* out) {
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < n; ++i) {
        float* o = out + i * f;
        if (rp[i] == rp[i + 1]) {
            for (int64_t j = 0; j < f; ++j) o[j] = 0.0f;
            continue;
        }
        for (int64_t j = 0; j < f; ++j) o[j] = -INFINITY;
        for (int32_t nz = rp[i]; nz < rp[i + 1]; ++nz) {
            const float* hj = h + (int64_t)ci[nz] * f;
            for (int64_t j = 0; j < f; ++j) o[j] = (o[j] < hj[j]) ? hj[j] : o[j];
        }
    }
}

/* The scalar tail of the fused SAGE dual matmul, layers.cpp:660-662:
 *   out += a_val * wn + h_val * ws
 * GCC's FMA contraction rewrites the inner sum as fma(a_val, wn, h_val*ws)
 * (the first product is fused into the addition, the second stays a plain
 * product), then adds it to out. */
static inline float sage_tail(float out, float a, float wn, float h, float ws) {
    return out + fmaf(a, wn, h * ws);
}

/* layers.cpp:538-752  SAGELayer::forward (fused aggregation + dual matmul)
 *   Mean (:587-673): agg = sum of neighbour rows (plain adds, nz order),
 *     deg = row length, agg *= 1.0f/deg when deg > 0.
 *   Max  (:674-734): agg = element-wise max, 0 for empty rows.
 *   dual matmul (:643-669): for each fi, for fo in the 8-wide part
 *     out = fma(agg_fi, Wn[fi,fo], out); out = fma(h_fi, Ws[fi,fo], out);
 *     the tail (fo >= 8*floor(F_out/8)) uses sage_tail().
 *   then add_bias (:738-740) and ReLU (:743-749).
 */
void or_sage_forward(int64_t n, int64_t f_in, int64_t f_out, int agg,
                     const int32_t* rp, const int32_t* ci, const float* h,
                     const float* w_neigh, const float* w_self,
                     const float* bias, int use_bias, int act, float* out) {
    memset(out, 0, (size_t)(n * f_out) * sizeof(float));
    const int64_t f8 = (f_out / 8) * 8;
    #pragma omp parallel
    {
        float* agg_row = (float*)malloc((size_t)(f_in > 0 ? f_in : 1) * sizeof(float));
        #pragma omp for schedule(dynamic, 64)
        for (int64_t i = 0; i < n; ++i) {
            const int32_t b = rp[i], e = rp[i + 1];
            for (int64_t f = 0; f < f_in; ++f) agg_row[f] = 0.0f;
            if (agg == 0) {
                const float deg = (float)(e - b);
                for (int32_t nz = b; nz < e; ++nz) {
                    const float* hj = h + (int64_t)ci[nz] * f_in;
                    for (int64_t f = 0; f < f_in; ++f) agg_row[f] += hj[f];
                }
                if (deg > 0.0f) {
                    const float inv = 1.0f / deg;
                    for (int64_t f = 0; f < f_in; ++f) agg_row[f] *= inv;
                }
            } else if (b < e) {
                for (int64_t f = 0; f < f_in; ++f) agg_row[f] = -INFINITY;
                for (int32_t nz = b; nz < e; ++nz) {
                    const float* hj = h + (int64_t)ci[nz] * f_in;
                    for (int64_t f = 0; f < f_in; ++f)
                        agg_row[f] = (agg_row[f] < hj[f]) ? hj[f] : agg_row[f];
                }
            }
            float* oi = out + i * f_out;
            const float* hi = h + i * f_in;
            for (int64_t fi = 0; fi < f_in; ++fi) {
                const float a = agg_row[fi], hv = hi[fi];
                const float* wn = w_neigh + fi * f_out;
                const float* ws = w_self + fi * f_out;
                for (int64_t fo = 0; fo < f8; ++fo) {
                    float o = fmaf(a, wn[fo], oi[fo]);
                    oi[fo] = fmaf(hv, ws[fo], o);
                }
                for (int64_t fo = f8; fo < f_out; ++fo)
                    oi[fo] = sage_tail(oi[fo], a, wn[fo], hv, ws[fo]);
            }
        }
        free(agg_row);
    }
    if (use_bias) or_add_bias(n, f_out, out, bias);
    if (act == 1) or_relu(n * f_out, out);
}

/* layers.cpp:286-339  GCNLayer::forward: matmul, spmm, add_bias, ReLU. */
void or_gcn_forward(int64_t n, int64_t f_in, int64_t f_out,
                    const int32_t* rp, const int32_t* ci, const float* av,
                    const float* h, const float* w, const float* bias,
                    int use_bias, int act, float* out) {
    float* hw = (float*)malloc((size_t)(n * f_out > 0 ? n * f_out : 1) * sizeof(float));
    or_matmul(n, f_in, f_out, h, w, hw);
    or_spmm(n, f_out, rp, ci, av, hw, out);
    free(hw);
    if (use_bias) or_add_bias(n, f_out, out, bias);
    if (act == 1) or_relu(n * f_out, out);
}

/* layers.cpp:991-1026  per-node attention dots.  Lane l of the 8-wide AVX2
 * accumulator holds fma-chains over f = l, l+8, ... < 8*floor(F/8)
 * (:1002-1008); the lanes are then added to 0.0f in lane order
 * (:1010-1013).  The scalar tail (:1014-1017) is what GCC 11 emits for it at
 * -O3 -mavx2 -mfma: tail elements are taken four at a time as a separate
 * multiply and add (the loop is vectorised over the (s, d) pair, which
 * keeps the products unfused), and the last (tail mod 4) elements are
 * contracted to fma.  Pinned bit-for-bit against the compiled reference for
 * F = 2..17, 41 and 100. */
void or_gat_scores(int64_t n, int64_t f, const float* wh, const float* al,
                   const float* ar, float* src, float* dst) {
    const int64_t f8 = (f / 8) * 8;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float* w = wh + i * f;
        float ls[8] = {0}, ld[8] = {0};
        for (int64_t q = 0; q < f8; q += 8)
            for (int l = 0; l < 8; ++l) {
                ls[l] = fmaf(al[q + l], w[q + l], ls[l]);
                ld[l] = fmaf(ar[q + l], w[q + l], ld[l]);
            }
        float s = 0.0f, d = 0.0f;
        for (int l = 0; l < 8; ++l) { s += ls[l]; d += ld[l]; }
        const int64_t t4 = f8 + ((f - f8) / 4) * 4;
        for (int64_t q = f8; q < t4; ++q) {
            s = s + al[q] * w[q];
            d = d + ar[q] * w[q];
        }
        for (int64_t q = t4; q < f; ++q) {
            s = fmaf(al[q], w[q], s);
            d = fmaf(ar[q], w[q], d);
        }
        src[i] = s;
        dst[i] = d;
    }
}

/* layers.cpp:945-1129  GATLayer::forward (fused SDDMM + softmax + SpMM)
 *   Wh = matmul(H, W)                                          :982
 *   scores                                                     :991-1026
 *   per row i (:1056-1111): e = s_i + d_j; e = e >= 0 ? e : slope*e;
 *   max; t = expf(e - max); sequential sum; inv = sum > 0 ? 1/sum : 0;
 *   alpha = t * inv; out_i = fma(alpha, Wh_j, out_i) in nz order.
 *   empty rows stay 0; then add_bias and ReLU.
 */
void or_gat_forward(int64_t n, int64_t f_in, int64_t f_out,
                    const int32_t* rp, const int32_t* ci, const float* h,
                    const float* w, const float* al, const float* ar,
                    const float* bias, float slope, int use_bias, int act,
                    float* out) {
    const size_t nf = (size_t)(n * f_out > 0 ? n * f_out : 1);
    float* wh = (float*)malloc(nf * sizeof(float));
    float* src = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    float* dst = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    or_matmul(n, f_in, f_out, h, w, wh);
    or_gat_scores(n, f_out, wh, al, ar, src, dst);
    memset(out, 0, (size_t)(n * f_out) * sizeof(float));
    int32_t max_deg = 0;
    for (int64_t i = 0; i < n; ++i)
        if (rp[i + 1] - rp[i] > max_deg) max_deg = rp[i + 1] - rp[i];
    #pragma omp parallel
    {
        float* attn = (float*)malloc((size_t)(max_deg > 0 ? max_deg : 1) * sizeof(float));
        #pragma omp for schedule(dynamic, 64)
        for (int64_t i = 0; i < n; ++i) {
            const int32_t b = rp[i], e = rp[i + 1];
            if (b == e) continue;
            const float si = src[i];
            const int32_t len = e - b;
            float mx = -INFINITY;
            for (int32_t t = 0; t < len; ++t) {
                float x = si + dst[ci[b + t]];
                x = (x >= 0.0f) ? x : slope * x;
                attn[t] = x;
                mx = (mx < x) ? x : mx;
            }
            float s = 0.0f;
            for (int32_t t = 0; t < len; ++t) {
                const float x = expf(attn[t] - mx);
                attn[t] = x;
                s += x;
            }
            const float inv = (s > 0.0f) ? (1.0f / s) : 0.0f;
            for (int32_t t = 0; t < len; ++t) attn[t] *= inv;
            float* oi = out + i * f_out;
            for (int32_t t = 0; t < len; ++t) {
                const float a = attn[t];
                const float* wj = wh + (int64_t)ci[b + t] * f_out;
                for (int64_t q = 0; q < f_out; ++q) oi[q] = fmaf(a, wj[q], oi[q]);
            }
        }
        free(attn);
    }
    free(wh);
    free(src);
    free(dst);
    if (use_bias) or_add_bias(n, f_out, out, bias);
    if (act == 1) or_relu(n * f_out, out);
}

/* ------------------------------------------------------------------------
 * graph_loader.cpp:14-206  CSV parsing, over an in-memory text.
 *   read_lines  :38-53   std::getline at '\n', trim " \t\r\n", skip empty
 *   is_header   :24-33   a letter or '_' before the first ',' ' ' '\t'
 *   parse_edges :61-107  first ',' splits; std::stoi of both sides
 *   parse_features :112-206  std::getline(ss, token, ','); stoi(trim(id)),
 *               stof(trim(feature)); the first data line fixes the count;
 *               rows placed by node_id, later lines overwriting earlier
 * std::stoi / std::stof are libstdc++'s: strtol(c_str, &end, 10) /
 * strtof(c_str, &end); nothing converted -> invalid_argument, errno ERANGE
 * (or a long outside int for stoi) -> out_of_range.  Fields are copied into
 * NUL-terminated buffers, so a NUL byte ends them as it ends c_str().
 * All errors are std::runtime_error in the reference (return 2 here).
 * ------------------------------------------------------------------------ */
typedef struct {
    int64_t b, e;
} or_span;

static int or_is_trim(unsigned char c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n'; }

/* Non-empty trimmed lines; *count receives their number.  Caller frees. */
static or_span* or_read_lines(const char* t, int64_t n, int64_t* count) {
    int64_t cap = 1;
    for (int64_t i = 0; i < n; ++i) cap += t[i] == '\n';
    or_span* s = (or_span*)malloc(sizeof(or_span) * (size_t)cap);
    int64_t k = 0, b = 0;
    while (b < n) {
        const char* nl = (const char*)memchr(t + b, '\n', (size_t)(n - b));
        int64_t e = nl ? (int64_t)(nl - t) : n;
        const int64_t next = nl ? e + 1 : n;
        int64_t lb = b, le = e;
        while (lb < le && or_is_trim((unsigned char)t[lb])) ++lb;
        while (le > lb && or_is_trim((unsigned char)t[le - 1])) --le;
        if (lb < le) {
            s[k].b = lb;
            s[k].e = le;
            ++k;
        }
        b = next;
    }
    *count = k;
    return s;
}

static int or_is_header(const char* t, or_span s) {
    for (int64_t p = s.b; p < s.e; ++p) {
        const unsigned char c = (unsigned char)t[p];
        if (c == ',' || c == ' ' || c == '\t') break;
        if (((c | 0x20) >= 'a' && (c | 0x20) <= 'z') || c == '_') return 1;
    }
    return 0;
}

/* [b, e) as a NUL-terminated copy; trimmed of " \t\r\n" when trim != 0. */
static char* or_field(const char* t, int64_t b, int64_t e, int trim) {
    if (trim) {
        while (b < e && or_is_trim((unsigned char)t[b])) ++b;
        while (e > b && or_is_trim((unsigned char)t[e - 1])) --e;
    }
    char* f = (char*)malloc((size_t)(e - b) + 1);
    memcpy(f, t + b, (size_t)(e - b));
    f[e - b] = '\0';
    return f;
}

static int or_stoi(const char* s, int32_t* out) {
    char* end;
    errno = 0;
    const long v = strtol(s, &end, 10);
    if (end == s) return 1;
    if (errno == ERANGE || v < INT_MIN || v > INT_MAX) return 2;
    *out = (int32_t)v;
    return 0;
}

static int or_stof(const char* s, float* out) {
    char* end;
    errno = 0;
    const float v = strtof(s, &end);
    if (end == s) return 1;
    if (errno == ERANGE) return 2;
    *out = v;
    return 0;
}

/* Appends the first `len` bytes of t[b..] (NULs included) to msg. */
static void or_err_line(const char* prefix, const char* t, int64_t b, int64_t e,
                        const char* suffix) {
    size_t k = (size_t)snprintf(g_err, sizeof g_err, "%s", prefix);
    for (int64_t p = b; p < e && k + 1 < sizeof g_err; ++p) g_err[k++] = t[p];
    g_err[k < sizeof g_err ? k : sizeof g_err - 1] = '\0';
    strncat(g_err, suffix, sizeof g_err - strlen(g_err) - 1);
}

int or_parse_edges(const char* text, int64_t n, const char* name, int32_t* src,
                   int32_t* dst, int64_t cap, int64_t* n_out) {
    int64_t nl;
    or_span* L = or_read_lines(text, n, &nl);
    int rc = 0;
    int64_t cnt = 0;
    if (nl == 0) {
        snprintf(g_err, sizeof g_err, "GraphLoader::parse_edges: file is empty: '%s'", name);
        rc = 2;
        goto done;
    }
    for (int64_t i = or_is_header(text, L[0]); i < nl; ++i) {
        const char* c = (const char*)memchr(text + L[i].b, ',', (size_t)(L[i].e - L[i].b));
        char pre[128];
        if (!c) {
            snprintf(pre, sizeof pre, "GraphLoader::parse_edges: malformed line %lld: '",
                     (long long)(i + 1));
            or_err_line(pre, text, L[i].b, L[i].e, "'");
            rc = 2;
            goto done;
        }
        const int64_t ci = (int64_t)(c - text);
        char* f1 = or_field(text, L[i].b, ci, 0);
        char* f2 = or_field(text, ci + 1, L[i].e, 0);
        int32_t s = 0, d = 0;
        const int r1 = or_stoi(f1, &s);
        const int r2 = r1 ? 0 : or_stoi(f2, &d);
        free(f1);
        free(f2);
        if (r1 || r2) {
            snprintf(pre, sizeof pre, "GraphLoader::parse_edges: invalid integer on line %lld: '",
                     (long long)(i + 1));
            or_err_line(pre, text, L[i].b, L[i].e, "'");
            rc = 2;
            goto done;
        }
        if (s < 0 || d < 0) {
            snprintf(g_err, sizeof g_err,
                     "GraphLoader::parse_edges: negative node ID on line %lld: src=%d, dst=%d",
                     (long long)(i + 1), s, d);
            rc = 2;
            goto done;
        }
        if (cnt < cap) {
            src[cnt] = s;
            dst[cnt] = d;
        }
        ++cnt;
    }
done:
    free(L);
    *n_out = cnt;
    return rc;
}

int or_parse_features(const char* text, int64_t n, const char* name, float* out,
                      int64_t cap, int64_t* rows_out, int64_t* cols_out) {
    int64_t nl;
    or_span* L = or_read_lines(text, n, &nl);
    int rc = 0;
    int64_t num_features = 0, nd = 0;
    int32_t max_id = -1;
    int32_t* ids = NULL;
    float* feats = NULL;
    *rows_out = 0;
    *cols_out = 0;
    if (nl == 0) {
        snprintf(g_err, sizeof g_err, "GraphLoader::parse_features: file is empty: '%s'", name);
        rc = 2;
        goto done;
    }
    const int64_t start = or_is_header(text, L[0]);
    nd = nl - start;
    if (nd == 0) {
        snprintf(g_err, sizeof g_err, "GraphLoader::parse_features: no data rows in '%s'", name);
        rc = 2;
        goto done;
    }
    ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)nd);
    size_t fcap = 1024, fused = 0;
    feats = (float*)malloc(sizeof(float) * fcap);
    for (int64_t i = start; i < nl; ++i) {
        char pre[160];
        /* first token: node_id */
        int64_t p = L[i].b;
        const char* c = (const char*)memchr(text + p, ',', (size_t)(L[i].e - p));
        int64_t te = c ? (int64_t)(c - text) : L[i].e;
        char* tok = or_field(text, p, te, 1);
        int32_t id = 0;
        const int r = or_stoi(tok, &id);
        free(tok);
        if (r) {
            snprintf(pre, sizeof pre, "GraphLoader::parse_features: invalid node_id on line %lld: '",
                     (long long)(i + 1));
            or_err_line(pre, text, p, te, "'");
            rc = 2;
            goto done;
        }
        if (id < 0) {
            snprintf(g_err, sizeof g_err, "GraphLoader::parse_features: negative node_id on line %lld",
                     (long long)(i + 1));
            rc = 2;
            goto done;
        }
        if (id > max_id) max_id = id;
        p = c ? te + 1 : L[i].e;
        int64_t k = 0;
        const size_t row0 = fused;
        while (p < L[i].e) { /* std::getline(ss, token, ',') until nothing is left */
            c = (const char*)memchr(text + p, ',', (size_t)(L[i].e - p));
            te = c ? (int64_t)(c - text) : L[i].e;
            tok = or_field(text, p, te, 1);
            float v = 0.0f;
            const int rf = or_stof(tok, &v);
            free(tok);
            if (rf) {
                snprintf(pre, sizeof pre,
                         "GraphLoader::parse_features: invalid feature on line %lld: '",
                         (long long)(i + 1));
                or_err_line(pre, text, p, te, "'");
                rc = 2;
                goto done;
            }
            if (fused == fcap) {
                fcap *= 2;
                feats = (float*)realloc(feats, sizeof(float) * fcap);
            }
            feats[fused++] = v;
            ++k;
            p = c ? te + 1 : L[i].e;
        }
        if (num_features == 0) {
            num_features = k;
            if (num_features == 0) {
                snprintf(g_err, sizeof g_err, "GraphLoader::parse_features: no features on line %lld",
                         (long long)(i + 1));
                rc = 2;
                goto done;
            }
        } else if (k != num_features) {
            snprintf(g_err, sizeof g_err,
                     "GraphLoader::parse_features: inconsistent feature count on line %lld: "
                     "expected %lld but got %lld",
                     (long long)(i + 1), (long long)num_features, (long long)k);
            rc = 2;
            goto done;
        }
        (void)row0;
        ids[i - start] = id;
    }
    {
        const int64_t rows = (int64_t)max_id + 1;
        *rows_out = rows;
        *cols_out = num_features;
        if (out && cap >= rows * num_features) {
            memset(out, 0, sizeof(float) * (size_t)(rows * num_features));
            for (int64_t d = 0; d < nd; ++d)
                memcpy(out + (int64_t)ids[d] * num_features, feats + d * num_features,
                       sizeof(float) * (size_t)num_features);
        }
    }
done:
    free(ids);
    free(feats);
    free(L);
    return rc;
}
