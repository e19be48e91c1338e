// sage.hip -- GraphSAGE on gfx950 (replaces SAGELayer::forward, reference
// src/layers.cpp:538-752, and sage_max_aggregate, :359-435).
//
// Two dataflows for out = act(AGG * Wn + H * Ws + b):
//   * concat: AGG = mean (or max) of the neighbour rows of H at width f_in,
//     then one dual GEMM over [AGG | H] x [Wn ; Ws].  With the in-order GEMM
//     this is the reference's own operation sequence (aggregation by plain
//     adds in nonzero order, x 1/deg, then the interleaved fma chain), so it
//     is bit-identical for rows handled as one chunk;
//   * transform first (mean only): T = H * [Ws | Wn] (one GEMM, 2 f_out
//     columns), then out = mean_j T_n[j] + T_s[i] + b in the aggregation's
//     epilogue.  Mean commutes with the linear map, so this is the same
//     function with fewer gathered bytes when f_out < f_in (regrouped
//     rounding: within tolerance, not bit-identical).
#include "aggregate.hpp"
#include "common.hpp"
#include "dense.hpp"
#include "spmm_plan.hpp"

#include <algorithm>

namespace tg {

namespace {

int resolve_dataflow(int dataflow, int agg, int64_t f_in, int64_t f_out, int64_t nnz) {
    if (dataflow != TG_SAGE_AUTO) return dataflow;
    if (agg != TG_AGG_MEAN || f_out >= f_in) return TG_SAGE_CONCAT;
    // Small graphs keep the reference's (bit-exact) dataflow.
    return nnz * f_in >= (int64_t(1) << 26) ? TG_SAGE_TRANSFORM_FIRST : TG_SAGE_CONCAT;
}

size_t sage_ws(int64_t n, int64_t f_in, int64_t f_out, int dataflow) {
    Carver c(nullptr, 0);
    if (dataflow == TG_SAGE_TRANSFORM_FIRST) {
        const int64_t fp = gather_pitch(f_out);
        c.take<float>(n * 2 * fp);
        c.take<float>(f_in * 2 * fp);
    } else {
        // the aggregate, and a copy of H, at a 4-float pitch (128-bit gathers)
        const int64_t fp = round_up(f_in, 4);
        c.take<float>(n * fp);
        c.take<float>(n * std::max(fp, ceil_div(f_in, 32) * 32));
    }
    return c.bytes();
}

}  // namespace

void sage_aggregate(const tg_spmm_plan_s& p, int64_t f, int agg, const int32_t* ci,
                    const float* h, int64_t ldh, float* out, int64_t ldo, hipStream_t s,
                    const BlockedCSR* blocked) {
    require(agg == TG_AGG_MEAN || agg == TG_AGG_MAX, "SAGELayer: unknown aggregator");
    AggEpilogue epi;
    epi.mean = agg == TG_AGG_MEAN;
    epi.max = agg == TG_AGG_MAX;
    if (blocked && agg == TG_AGG_MEAN) {
        run_aggregate_blocked(*blocked, f, h, ldh, out, ldo, epi, s);
    } else {
        epi.long_rows = p.precision == TG_PRECISION_EXACT;  // split rows as in-order chains
        run_aggregate(p, f, ci, nullptr, h, ldh, out, ldo, epi, s);
    }
}

int sage_dataflow_for(int dataflow, int agg, int64_t f_in, int64_t f_out, int64_t nnz) {
    return resolve_dataflow(dataflow, agg, f_in, f_out, nnz);
}

bool sage_tf_tiled(int64_t f_out, bool blocked) { return blocked && gather_pitch(f_out) % 32 == 0; }

int64_t sage_tf_floats(int64_t n, int64_t f_out) { return n * 2 * gather_pitch(f_out); }

void sage_transform(int64_t n, int64_t f_in, int64_t f_out, const float* h, const float* wn,
                    const float* ws, bool tiled, float* t, float* wcat, hipStream_t s,
                    int gemm_algo) {
    // [Ws | 0 | Wn | 0]: each half padded to fp = gather_pitch(f_out)
    // columns, so the neighbour half's rows start line-aligned and are
    // gathered with 128-bit loads; the zero columns make the GEMM write
    // zeros into the padding.
    const int64_t fp = gather_pitch(f_out);
    if (fp != f_out) fill_zero_2d(wcat, f_in, 2 * fp, 2 * fp, s);
    TG_HIP(hipMemcpy2DAsync(wcat, 2 * fp * sizeof(float), ws, f_out * sizeof(float),
                            f_out * sizeof(float), f_in, hipMemcpyDeviceToDevice, s));
    TG_HIP(hipMemcpy2DAsync(wcat + fp, 2 * fp * sizeof(float), wn, f_out * sizeof(float),
                            f_out * sizeof(float), f_in, hipMemcpyDeviceToDevice, s));
    // The blocked passes gather T tile-major (32-column tiles of n rows
    // each, the GEMM's store layout): a tile's rows are one contiguous
    // slab instead of lines 2 fp floats apart.
    GemmArgs g;
    g.m = n;
    g.n = 2 * fp;
    g.a1 = h;
    g.lda1 = f_in;
    g.b1 = wcat;
    g.ldb1 = 2 * fp;
    g.k1 = f_in;
    g.c = t;
    g.ldc = tiled ? 32 : 2 * fp;
    g.c_tile_stride = tiled ? n * 32 : 0;
    gemm(g, gemm_algo, s);
}

size_t sage_forward_ws(int64_t n, int64_t f_in, int64_t f_out, int agg, int dataflow,
                       int64_t nnz) {
    return sage_ws(n, f_in, f_out, resolve_dataflow(dataflow, agg, f_in, f_out, nnz));
}

void sage_forward(const tg_spmm_plan_s& p, int64_t n, int64_t f_in, int64_t f_out, int agg,
                  const int32_t* ci, const float* h, const float* wn, const float* ws,
                  const float* bias, int act, int post, int dataflow, float* out, void* work,
                  size_t work_bytes, hipStream_t s, int gemm_algo,
                  const BlockedCSR* blocked, const float* t_pre) {
    require(n == p.m, "SAGELayer::forward: plan rows differ from n");
    require(f_in >= 0 && f_out >= 0, "SAGELayer::forward: negative size");
    require(act == TG_ACT_NONE || act == TG_ACT_RELU, "SAGELayer: unknown activation");
    require(post >= TG_POST_NONE && post <= TG_POST_ELU, "SAGELayer: unknown post activation");
    if (n == 0 || f_out == 0) return;
    const int64_t nnz = p.nnz_bound;
    dataflow = resolve_dataflow(dataflow, agg, f_in, f_out, nnz);
    require(dataflow == TG_SAGE_CONCAT || dataflow == TG_SAGE_TRANSFORM_FIRST,
            "SAGELayer: unknown dataflow");
    require(dataflow == TG_SAGE_CONCAT || agg == TG_AGG_MEAN,
            "SAGELayer: transform-first needs the mean aggregator");
    DeviceBuffer own;
    if (work == nullptr) {
        own.resize(sage_ws(n, f_in, f_out, dataflow));
        work = own.get();
        work_bytes = own.size();
    }
    Carver c(work, work_bytes);
    if (dataflow == TG_SAGE_CONCAT) {
        // H at a row pitch of a multiple of 4 floats (a copy when f_in is
        // not): the aggregation gathers 128-bit vectors and stores the
        // aggregate at the same pitch; the padding is loaded, never stored.
        const int64_t fp = round_up(f_in, 4);
        float* aggb = c.take<float>(n * fp);
        const float* hg = h;
        if (blocked && agg == TG_AGG_MEAN) {
            // tile-major copy of H for the blocked passes
            const int64_t nt = ceil_div(f_in, 32);
            float* ht = c.take<float>(n * nt * 32);
            for (int64_t t = 0; t < nt; ++t)
                TG_HIP(hipMemcpy2DAsync(ht + t * n * 32, 32 * sizeof(float), h + t * 32,
                                        f_in * sizeof(float),
                                        std::min<int64_t>(32, f_in - t * 32) * sizeof(float), n,
                                        hipMemcpyDeviceToDevice, s));
            AggEpilogue epi;
            epi.mean = 1;
            epi.b_tile_stride = n * 32;
            run_aggregate_blocked(*blocked, f_in, ht, 32, aggb, fp, epi, s);
        } else {
            if (fp != f_in) {
                float* hp = c.take<float>(n * fp);
                TG_HIP(hipMemcpy2DAsync(hp, fp * sizeof(float), h, f_in * sizeof(float),
                                        f_in * sizeof(float), n, hipMemcpyDeviceToDevice, s));
                hg = hp;
            }
            sage_aggregate(p, f_in, agg, ci, hg, fp, aggb, fp, s, blocked);
        }
        GemmArgs g;
        g.m = n;
        g.n = f_out;
        g.a1 = aggb;
        g.lda1 = fp;
        g.b1 = wn;
        g.ldb1 = f_out;
        g.k1 = f_in;
        g.a2 = hg;
        g.lda2 = hg == h ? f_in : fp;
        g.b2 = ws;
        g.ldb2 = f_out;
        g.k2 = f_in;
        g.c = out;
        g.ldc = f_out;
        g.bias = bias;
        g.epi = act == TG_ACT_RELU ? TG_EPI_RELU : TG_EPI_NONE;
        g.tail_from = (f_out / 8) * 8;  // the reference's scalar tail columns
        gemm(g, gemm_algo, s);
        add_bias_act(out, n, f_out, f_out, nullptr, TG_ACT_NONE, post, s);
    } else {
        const int64_t fp = gather_pitch(f_out);
        float* t = c.take<float>(n * 2 * fp);
        float* wcat = c.take<float>(f_in * 2 * fp);
        const bool tiled = sage_tf_tiled(f_out, blocked != nullptr);
        if (t_pre != nullptr)
            t = const_cast<float*>(t_pre);  // (read only from here on)
        else
            sage_transform(n, f_in, f_out, h, wn, ws, tiled, t, wcat, s, gemm_algo);
        AggEpilogue epi;
        epi.mean = 1;
        epi.self = t;
        epi.ld_self = tiled ? 32 : 2 * fp;
        epi.self_tile_stride = tiled ? n * 32 : 0;
        epi.bias = bias;
        epi.act = act;
        epi.post = post;
        if (tiled) {
            epi.b_tile_stride = n * 32;
            epi.mask_tail = 1;
            run_aggregate_blocked(*blocked, f_out, t + (fp / 32) * n * 32, 32, out, f_out, epi, s);
        } else if (blocked) {
            run_aggregate_blocked(*blocked, f_out, t + fp, 2 * fp, out, f_out, epi, s);
        } else {
            epi.long_rows = p.precision == TG_PRECISION_EXACT;
            run_aggregate(p, f_out, ci, nullptr, t + fp, 2 * fp, out, f_out, epi, s);
        }
    }
    if (own.get()) TG_HIP(hipStreamSynchronize(s));
}

}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_sage_aggregate(tg_spmm_plan_t plan, int64_t n, int64_t f, int agg,
                      const int32_t* row_ptr, const int32_t* col_ind, const float* h,
                      int64_t ldh, float* out, int64_t ldo, tg_stream_t stream) {
    return guard([&] {
        require(plan != nullptr, "sage_aggregate: plan is null");
        require(row_ptr == plan->row_ptr, "sage_aggregate: row_ptr differs from the plan's");
        require(n == plan->m, "sage_aggregate: n differs from the plan's rows");
        tg::sage_aggregate(*plan, f, agg, col_ind, h, ldh, out, ldo,
                           static_cast<hipStream_t>(stream), nullptr);
    });
}

size_t tg_sage_forward_workspace_size(int64_t n, int64_t f_in, int64_t f_out, int agg,
                                      int dataflow, int64_t nnz) {
    return tg::sage_forward_ws(n, f_in, f_out, agg, dataflow, nnz);
}

int tg_sage_forward(tg_spmm_plan_t plan, int64_t n, int64_t f_in, int64_t f_out, int agg,
                    const int32_t* row_ptr, const int32_t* col_ind, const float* h,
                    const float* w_neigh, const float* w_self, const float* bias, int act,
                    int post, int dataflow, float* out, void* workspace, size_t workspace_bytes,
                    tg_stream_t stream) {
    return guard([&] {
        require(plan != nullptr, "SAGELayer::forward: plan is null");
        require(row_ptr == plan->row_ptr, "SAGELayer::forward: row_ptr differs from the plan's");
        tg::sage_forward(*plan, n, f_in, f_out, agg, col_ind, h, w_neigh, w_self, bias, act, post,
                         dataflow, out, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream), TG_GEMM_AUTO, nullptr, nullptr);
    });
}

}  // extern "C"
