// model.hip -- the sequential GNN execution graph on the device.
//
// Replaces tinygnn::Model (reference include/tinygnn/model.hpp:89-164,
// src/model.cpp:191-439): a registry of GCN / SAGE / GAT layers with the
// reference's constructor defaults and weight names, load_weights from a
// set of named tensors, and forward().
//
// forward() follows model.cpp:359-439: gcn_norm if any GCN layer,
// add_self_loops if any GAT layer, layers in order, multi-head GAT concat or
// average, then the post activation.  Differences of mapping, not of
// result:
//   * all heads of a GAT layer run as one GEMM + one fused edge kernel;
//   * GCN's bias/activation and the post activation are applied in the
//     aggregation's store;
//   * GCN and GAT share A + I's structure (gcn_norm's output has the
//     structure of add_self_loops' output; GAT reads structure only), so when
//     both are present the self-loop pass runs once;
//   * the GCN, SAGE-mean and GAT aggregations over large, dense graphs run
//     column blocked (blocked.hip):
//     one pass per block of source nodes, so the gathered rows of a pass
//     stay in L2; each pass continues the rows' sums, which keeps exact
//     precision's in-order sums when the rows are in block order;
//   * in fast precision, when every value of A + I is exactly 1 (A's values
//     all 1 and no diagonal in A, as an edge list's CSR), a blocked GCN
//     aggregation is factored: A_norm (HW) = D^-1/2 (A + I) (D^-1/2 HW),
//     the D^-1/2 on the right applied in the GEMM's store and the one on the
//     left in the aggregation's, so the passes read the column indices alone
//     (no values): the same sum, rounded differently;
//   * TG_FORWARD_CACHED keeps the preprocessed adjacency and the row plans
//     while the adjacency pointers, sizes, precision and layer list are
//     unchanged and tg_model_invalidate has not been called since;
//     TG_FORWARD_REFERENCE recomputes them on every call, as the reference.
#include "aggregate.hpp"
#include "common.hpp"
#include "dense.hpp"
#include "layers.hpp"
#include "spmm_plan.hpp"

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace {

using tg::DeviceBuffer;
using tg::require;

struct HostTensor {
    int64_t rows = 0, cols = 0;
    std::vector<float> data;
};

enum class LType { GCN, SAGE, GAT };

struct Layer {
    LType type;
    int64_t in = 0, out = 0, heads = 1;
    bool concat = true;
    float slope = 0.2f;
    bool bias = true;
    int act = TG_ACT_RELU;
    int post = TG_POST_NONE;
    int agg = TG_AGG_MEAN;
    DeviceBuffer w;       // GCN [in x out]; GAT [in x heads*out] (head-major columns)
    DeviceBuffer wn, ws;  // SAGE [in x out]
    DeviceBuffer b;       // [heads*out]
    DeviceBuffer al, ar;  // GAT [heads*out]

    int64_t out_cols() const { return type == LType::GAT && concat ? heads * out : out; }
    int64_t wide() const { return type == LType::GAT ? heads * out : out; }
};

void upload(DeviceBuffer& d, const std::vector<float>& h) {
    d.resize(h.size() * sizeof(float));
    if (!h.empty())
        TG_HIP(hipMemcpy(d.get(), h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
}

std::string shape(int64_t r, int64_t c) {
    return "(" + std::to_string(r) + "\xC3\x97" + std::to_string(c) + ")";
}

}  // namespace

struct tg_model_s {
    std::vector<Layer> layers;
    std::map<std::string, HostTensor> staged;
    int sage_dataflow = TG_SAGE_AUTO;
    int precision = TG_PRECISION_FAST;
    int built_precision = -1;  // precision the cached plans were built for
    int64_t block_rows = -1;   // column blocking (tg_model_set_blocking)
    bool direct_split = true;  // tg_model_set_self_loop_split
    bool resident = false;     // tg_model_set_resident_passes
    int64_t built_block_rows = -2;  // blocking the blocked copies were built for (-2: none)

    // bumped by every add_*_layer: the cached adjacency state (which of
    // A + I, its values, A's plan and the blocked copies exist, and the
    // feature width the plans were sized for) depends on the layer list
    uint64_t layers_gen = 0;
    uint64_t built_layers_gen = ~uint64_t(0);

    // adjacency-derived state
    bool have_cache = false;
    const int32_t* key_rp = nullptr;
    const int32_t* key_ci = nullptr;
    const float* key_v = nullptr;
    int64_t key_n = -1, key_nnz = -1;
    DeviceBuffer sl_rp, sl_ci, sl_v;  // A + I (normalised values when GCN is present)
    DeviceBuffer dis;                 // gcn_norm's 1/sqrt(deg) (GCN present)
    // fast precision, GCN present: every value of A + I is 1 (the blocked
    // GCN aggregation is factored, its blocked copy carries no values)
    bool unit_sl = false;
    // sl_v holds A + I's values (GCN present, unless only the factored
    // blocked path reads A + I)
    bool sl_values = false;
    // blk_sl was split from A directly with the diagonal placed per row, and
    // A + I itself (sl_rp, sl_ci, sl_v) was not written
    bool blk_sl_direct = false;
    // the last unit-value check's answer: while it was yes, the next check
    // is read after the direct split's own synchronisation (the split
    // assuming unit values, dropped when they are not) instead of before it
    bool unit_guess = true;
    DeviceBuffer flag;
    tg::PinnedBuffer flag_host;
    std::unique_ptr<tg_spmm_plan_s> plan_raw, plan_sl;
    bool plan_sl_built = false;  // plan_sl holds A + I's row plan (ensure_plan_sl)
    bool plan_raw_built = false;  // plan_raw holds A's row plan (ensure_plan_raw)
    // column-blocked copies for the large aggregations (fast precision):
    // A_norm for GCN, A's structure for SAGE-mean
    std::unique_ptr<tg::BlockedCSR> blk_sl, blk_raw;

    // per-forward buffers
    DeviceBuffer act[2], tmp, scores, work;

    // Layer 0's transform (X * W, for GAT also its scores), computed on a
    // side stream while the per-call preprocessing of the adjacency runs on
    // the caller's stream, which it synchronises; the caller's stream waits
    // for it before the aggregation (pre_*: its outputs)
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    DeviceBuffer pre, pre_w, pre_dis, pre_flag;
    // launches that transform; set during a reference-semantics call's
    // preprocessing, whose first blocked build calls it after its scatter
    // (BlockedCSR::after_split)
    std::function<void()> fork_hook;

    tg_model_s() = default;
    tg_model_s(const tg_model_s&) = delete;
    tg_model_s& operator=(const tg_model_s&) = delete;
    ~tg_model_s() {
        if (side) (void)hipStreamSynchronize(side);
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_join) (void)hipEventDestroy(ev_join);
        if (side) (void)hipStreamDestroy(side);
    }

    bool need_norm() const {
        for (auto& l : layers) if (l.type == LType::GCN) return true;
        return false;
    }
    bool need_sl() const {
        for (auto& l : layers) if (l.type == LType::GAT) return true;
        return false;
    }
    bool need_raw() const {
        for (auto& l : layers) if (l.type == LType::SAGE) return true;
        return false;
    }
    bool need_raw_mean() const {
        for (auto& l : layers) if (l.type == LType::SAGE && l.agg == TG_AGG_MEAN) return true;
        return false;
    }
    int64_t max_wide() const {
        int64_t m = 1;
        for (auto& l : layers) m = std::max({m, l.wide(), l.in, l.out_cols()});
        return m;
    }
};

namespace tg {
namespace {

// *flag = 0 if some value of A is not exactly 1 (*flag is 1 before).
// VEC = 4: 128-bit reads (v 16-byte aligned), the last nnz % 4 values on
// the first thread.
template <int VEC>
__global__ __launch_bounds__(256) void unit_values_kernel(const float* __restrict__ v,
                                                          int64_t nnz,
                                                          int32_t* __restrict__ flag) {
    bool bad = false;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if constexpr (VEC == 4) {
        const float4* v4 = reinterpret_cast<const float4*>(v);
        for (int64_t i = tid; i < nnz / 4; i += stride) {
            const float4 x = v4[i];
            bad |= (x.x != 1.0f) | (x.y != 1.0f) | (x.z != 1.0f) | (x.w != 1.0f);
        }
        if (tid == 0)
            for (int64_t i = nnz / 4 * 4; i < nnz; ++i) bad |= v[i] != 1.0f;
    } else {
        for (int64_t i = tid; i < nnz; i += stride) bad |= v[i] != 1.0f;
    }
    if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) *flag = 0;  // one store per wave
}

int64_t add_layer(tg_model_s& m, Layer&& l) {
    const char* name = l.type == LType::GCN ? "GCNLayer" : l.type == LType::SAGE ? "SAGELayer"
                                                                                 : "GATLayer";
    if (l.in <= 0) throw std::invalid_argument(std::string(name) + ": in_features must be > 0.");
    if (l.out <= 0) throw std::invalid_argument(std::string(name) + ": out_features must be > 0.");
    require(l.heads >= 1, "Model::add_gat_layer: num_heads must be >= 1");
    require(l.act == TG_ACT_NONE || l.act == TG_ACT_RELU, std::string(name) + ": unknown activation");
    require(l.post >= TG_POST_NONE && l.post <= TG_POST_ELU, "Model: unknown post activation");
    require(l.agg == TG_AGG_MEAN || l.agg == TG_AGG_MAX, "SAGELayer: unknown aggregator");
    // zero-initialised weights, as the reference's layer constructors
    const int64_t wide = l.type == LType::GAT ? l.heads * l.out : l.out;
    std::vector<float> zw(static_cast<size_t>(l.in * wide), 0.0f), zb(static_cast<size_t>(wide), 0.0f);
    if (l.type == LType::SAGE) {
        upload(l.wn, zw);
        upload(l.ws, zw);
    } else {
        upload(l.w, zw);
    }
    upload(l.b, zb);
    if (l.type == LType::GAT) {
        upload(l.al, zb);
        upload(l.ar, zb);
    }
    m.layers.push_back(std::move(l));
    ++m.layers_gen;  // the cached adjacency state no longer matches the layers
    return static_cast<int64_t>(m.layers.size()) - 1;
}

const HostTensor& get(const tg_model_s& m, const std::string& name) {
    auto it = m.staged.find(name);
    if (it == m.staged.end())
        throw std::runtime_error("Model::load_weights: missing tensor '" + name + "'");
    return it->second;
}

void check_shape(const HostTensor& t, int64_t r, int64_t c, const std::string& what) {
    if (t.rows != r || t.cols != c)
        throw std::invalid_argument(what + ": expected shape " + shape(r, c) + ", got " +
                                    shape(t.rows, t.cols) + ".");
}

void load_weights(tg_model_s& m) {
    for (size_t li = 0; li < m.layers.size(); ++li) {
        Layer& l = m.layers[li];
        const std::string p = "layer" + std::to_string(li);
        if (l.type == LType::GCN) {
            const HostTensor& w = get(m, p + ".weight");
            check_shape(w, l.in, l.out, "GCNLayer::set_weight");
            upload(l.w, w.data);
            if (l.bias) {
                const HostTensor& b = get(m, p + ".bias");
                check_shape(b, 1, l.out, "GCNLayer::set_bias");
                upload(l.b, b.data);
            }
        } else if (l.type == LType::SAGE) {
            const HostTensor& wn = get(m, p + ".weight_neigh");
            check_shape(wn, l.in, l.out, "SAGELayer::set_weight_neigh");
            const HostTensor& ws = get(m, p + ".weight_self");
            check_shape(ws, l.in, l.out, "SAGELayer::set_weight_self");
            upload(l.wn, wn.data);
            upload(l.ws, ws.data);
            if (l.bias) {
                const HostTensor& b = get(m, p + ".bias");
                check_shape(b, 1, l.out, "SAGELayer::set_bias");
                upload(l.b, b.data);
            }
        } else {
            const int64_t H = l.heads, F = l.out, wide = H * F;
            std::vector<float> w(static_cast<size_t>(l.in * wide)), al(wide), ar(wide),
                b(wide, 0.0f);
            for (int64_t h = 0; h < H; ++h) {
                const std::string hp = p + ".head" + std::to_string(h);
                const HostTensor& wh = get(m, hp + ".weight");
                check_shape(wh, l.in, F, "GATLayer::set_weight");
                const HostTensor& a_l = get(m, hp + ".attn_left");
                check_shape(a_l, 1, F, "GATLayer::set_attn_left");
                const HostTensor& a_r = get(m, hp + ".attn_right");
                check_shape(a_r, 1, F, "GATLayer::set_attn_right");
                for (int64_t r = 0; r < l.in; ++r)
                    for (int64_t c = 0; c < F; ++c) w[r * wide + h * F + c] = wh.data[r * F + c];
                for (int64_t c = 0; c < F; ++c) {
                    al[h * F + c] = a_l.data[c];
                    ar[h * F + c] = a_r.data[c];
                }
                if (l.bias) {
                    const HostTensor& bb = get(m, hp + ".bias");
                    check_shape(bb, 1, F, "GATLayer::set_bias");
                    for (int64_t c = 0; c < F; ++c) b[h * F + c] = bb.data[c];
                }
            }
            upload(l.w, w);
            upload(l.al, al);
            upload(l.ar, ar);
            upload(l.b, b);
        }
    }
}

// Column-blocked copies, built by cached-mode calls only (the build is paid
// once, not per call).  Exact precision keeps them only for structures whose
// rows are in block order, with plans that split no row: each row is then
// still one chain in nonzero order, continued across the passes.
void prepare_blocked(tg_model_s& m, int64_t n, int64_t nnz, const int32_t* rp,
                     const int32_t* ci, hipStream_t s) {
    // rebuilt in place: the blocked copies keep their buffers and plans
    m.built_block_rows = m.block_rows;
    const bool exact = m.precision == TG_PRECISION_EXACT;
    const int64_t maxf = m.max_wide();
    const int64_t chunk = exact ? (int64_t(1) << 24) : 0;
    // A + I: GCN's normalised values, or the structure alone for GAT (weighted
    // passes: 64-column lane groups); A: SAGE's mean (32-column groups)
    // (a factored GCN aggregation reads no values either).  Passes without a
    // value stream run in 32-column groups, as SAGE's (config-E GCN, factored:
    // 64-column groups at 10 blocks 9.64 ms, 32-column groups at 6 blocks
    // 9.36 ms).  GAT keeps 64-column groups: its passes compute a weight per
    // entry and lane group, and 32-column groups double that work (config-E
    // fast GAT, 32-column groups: 13.5-13.9 ms at 5-10 blocks against 12.0 ms).
    const int gc_sl = (m.unit_sl && !m.need_sl()) ? 32 : 64;
    const int64_t r_sl = resolve_block_rows(m.block_rows, n, nnz + n, gc_sl);
    if (m.blk_sl_direct) {
        // A + I's blocked copy was split from A by prepare_adjacency
    } else if ((m.need_norm() || m.need_sl()) && r_sl > 0) {
        if (!m.blk_sl) m.blk_sl = std::make_unique<BlockedCSR>();
        m.blk_sl->resident = m.resident && !exact && gc_sl == 32;  // the factored GCN's sums
        m.blk_sl->after_split = m.fork_hook;
        build_blocked(*m.blk_sl, n, nnz + n, m.sl_rp.as<int32_t>(), m.sl_ci.as<int32_t>(),
                      m.need_norm() && !m.unit_sl ? m.sl_v.as<float>() : nullptr, r_sl, maxf, s,
                      chunk);
        m.blk_sl->group_cols = gc_sl;
        if (exact && !m.blk_sl->in_order) m.blk_sl.reset();
    } else {
        m.blk_sl.reset();
    }
    const int64_t r_raw = resolve_block_rows(m.block_rows, n, nnz, 32);
    if (m.need_raw_mean() && r_raw > 0) {
        if (!m.blk_raw) m.blk_raw = std::make_unique<BlockedCSR>();
        m.blk_raw->resident = m.resident && !exact;  // SAGE's mean: plain sums
        m.blk_raw->after_split = m.fork_hook;
        build_blocked(*m.blk_raw, n, nnz, rp, ci, nullptr, r_raw, maxf, s, chunk);
        m.blk_raw->group_cols = 32;
        if (exact && !m.blk_raw->in_order) m.blk_raw.reset();
    } else {
        m.blk_raw.reset();
    }
}

// A + I's unblocked row plan, where something reads it: GAT (its statistics
// run over the plan's chunks) and an unblocked GCN aggregation.  A blocked
// GCN runs on the block plans alone (config-E reference-semantics GCN: one
// plan build and its synchronisation fewer per call).
void ensure_plan_sl(tg_model_s& m, int64_t n, int64_t nnz, hipStream_t s) {
    // (a blocked copy split from A directly serves every reader of A + I)
    const bool needed = !m.blk_sl_direct && (m.need_sl() || (m.need_norm() && !m.blk_sl));
    if (!needed || m.plan_sl_built) return;
    const int64_t chunk = m.precision == TG_PRECISION_EXACT ? (int64_t(1) << 24) : 0;
    build_plan(*m.plan_sl, n, nnz + n, m.sl_rp.as<int32_t>(), m.max_wide(), chunk, s);
    m.plan_sl_built = true;
}

// A's row plan, where something reads it: a SAGE layer whose aggregation
// does not block (SAGE-Max, or no blocked copy of A).  Blocked SAGE-mean
// layers run on the block plans alone (config-E reference-semantics SAGE:
// one plan build and its synchronisation fewer per call); the plan then
// carries only the sizes sage_forward checks.
void ensure_plan_raw(tg_model_s& m, int64_t n, int64_t nnz, const int32_t* rp, hipStream_t s) {
    if (!m.need_raw()) return;
    bool needed = m.blk_raw == nullptr;
    for (auto& l : m.layers)
        if (l.type == LType::SAGE && l.agg != TG_AGG_MEAN) needed = true;
    if (m.plan_raw_built) return;
    if (!needed) {
        m.plan_raw->m = n;
        m.plan_raw->nnz_bound = nnz;
        m.plan_raw->row_ptr = rp;
        m.plan_raw->precision = m.precision;
        return;
    }
    const int64_t chunk = m.precision == TG_PRECISION_EXACT ? (int64_t(1) << 24) : 0;
    build_plan(*m.plan_raw, n, nnz, rp, m.max_wide(), chunk, s);
    m.plan_raw->precision = m.precision;
    m.plan_raw_built = true;
}

// Whether the forward can keep the cached adjacency state (prepare_adjacency
// then rebuilds at most the blocked copies).
bool adjacency_cached(const tg_model_s& m, int64_t n, int64_t nnz, const int32_t* rp,
                      const int32_t* ci, const float* v, int mode) {
    const bool same = m.have_cache && m.key_rp == rp && m.key_ci == ci && m.key_v == v &&
                      m.key_n == n && m.key_nnz == nnz && m.built_precision == m.precision &&
                      m.built_layers_gen == m.layers_gen;
    // a new blocking setting keeps the cached state, unless A + I's values
    // were skipped for the factored path (an unblocked GCN needs them), or
    // A + I's blocked copy came straight from A (A + I was not written)
    const bool values_ok = (m.sl_values || !m.need_norm()) && !m.blk_sl_direct;
    return mode == TG_FORWARD_CACHED && same && (values_ok || m.built_block_rows == m.block_rows);
}

void prepare_adjacency(tg_model_s& m, int64_t n, int64_t nnz, const int32_t* rp,
                       const int32_t* ci, const float* v, int mode, hipStream_t s) {
    if (adjacency_cached(m, n, nnz, rp, ci, v, mode)) {
        // a cached call after a reference-mode one (or a new blocking
        // setting) adds the blocked copies to the state it reuses
        if (m.built_block_rows != m.block_rows) {
            prepare_blocked(m, n, nnz, rp, ci, s);
            if (m.need_norm() || m.need_sl()) ensure_plan_sl(m, n, nnz, s);
            ensure_plan_raw(m, n, nnz, rp, s);
        }
        return;
    }
    m.have_cache = false;
    m.built_block_rows = -2;  // the blocked copies are rebuilt below
    const int64_t maxf = m.max_wide();
    // exact: no row is split, so every row is one fma chain in nonzero order
    const int64_t chunk = m.precision == TG_PRECISION_EXACT ? (int64_t(1) << 24) : 0;
    // plans and buffers are rebuilt in place (they only grow), so a forward
    // with the reference's per-call preprocessing allocates nothing once warm
    // A's row plan is built by ensure_plan_raw, once the blocking is known
    if (m.need_raw()) {
        if (!m.plan_raw) m.plan_raw = std::make_unique<tg_spmm_plan_s>();
        m.plan_raw_built = false;
    } else {
        m.plan_raw.reset();
    }
    m.unit_sl = false;
    m.sl_values = false;
    m.blk_sl_direct = false;
    if (m.need_norm() || m.need_sl()) {
        require(nnz + n < (int64_t(1) << 31), "Model::forward: nnz + n must be < 2^31");
        m.work.reserve(self_loops_workspace(n));
        m.flag.reserve(sizeof(int32_t));
        m.flag_host.reserve(2 * sizeof(int32_t));
        int32_t* host = m.flag_host.as<int32_t>();
        // the blocking prepare_blocked resolves for a unit A + I
        const int gc_unit = m.need_sl() ? 64 : 32;
        const int64_t r_unit = resolve_block_rows(m.block_rows, n, nnz + n, gc_unit);
        const bool will_block = r_unit > 0;
        // fast precision, blocked: all of A's values exactly 1?  Then, with
        // no diagonal in A, every value of A + I is 1 and the blocked GCN
        // aggregation is factored (it reads no values); unblocked, the
        // check and its synchronisation are skipped
        bool unit_v = false;
        // the check's answer read after the direct split (below), which
        // then assumes unit values (GCN without GAT, the direct split on,
        // and the last check said yes): one synchronisation and the launch
        // gaps after it fewer per call
        bool unit_late = false;
        if (m.need_norm() && m.precision != TG_PRECISION_EXACT && will_block) {
            fill_i32(m.flag.as<int32_t>(), 1, 1, s);
            const int64_t blocks =
                std::min<int64_t>(std::max<int64_t>(ceil_div(nnz, 1024), 1), 4096);
            if (reinterpret_cast<uintptr_t>(v) % 16 == 0)
                unit_values_kernel<4><<<static_cast<unsigned>(blocks), 256, 0, s>>>(
                    v, nnz, m.flag.as<int32_t>());
            else
                unit_values_kernel<1><<<static_cast<unsigned>(blocks), 256, 0, s>>>(
                    v, nnz, m.flag.as<int32_t>());
            TG_LAUNCH_CHECK();
            TG_HIP(hipMemcpyAsync(host, m.flag.as<int32_t>(), sizeof(int32_t),
                                  hipMemcpyDeviceToHost, s));
            unit_late = m.unit_guess && m.direct_split && !m.need_sl();
            if (!unit_late) {
                TG_HIP(hipStreamSynchronize(s));
                unit_v = host[0] == 1;
                m.unit_guess = unit_v;
            }
        }
        // A + I's values: GAT reads the structure alone; GCN needs the
        // normalised values unless its aggregation will run factored
        // GAT layers in fast precision whose softmax rides along the blocked
        // passes read A + I's structure only through its blocked copy
        bool gat_online = m.precision != TG_PRECISION_EXACT && !m.need_norm();
        for (auto& l : m.layers)
            if (l.type == LType::GAT && !gat_blocked_ok(l.heads, l.out, l.concat))
                gat_online = false;
        const bool gcn_direct = (unit_v || unit_late) && !m.need_sl();
        const bool gat_direct = m.need_sl() && gat_online;
        if (m.direct_split && will_block && (gcn_direct || gat_direct)) {
            // Only blocked passes without values read A + I (the factored
            // GCN, or GAT carrying its softmax): the blocked copy is split
            // from A directly, each row's diagonal placed where
            // add_self_loops inserts it, and the GCN's dis comes from the
            // row lengths; A + I itself is never written (config-E
            // reference-semantics GCN 10.30 -> 9.80 ms).  Valid for sorted
            // rows of A without a diagonal, which the build checks;
            // otherwise the path below.
            host[1] = 0;
            if (gcn_direct) {
                m.dis.reserve(n * sizeof(float));
                fill_i32(m.flag.as<int32_t>(), 1, 0, s);
                unit_self_loop_dis(n, rp, m.dis.as<float>(), m.flag.as<int32_t>(), s);
                TG_HIP(hipMemcpyAsync(host + 1, m.flag.as<int32_t>(), sizeof(int32_t),
                                      hipMemcpyDeviceToHost, s));
            }
            if (!m.blk_sl) m.blk_sl = std::make_unique<BlockedCSR>();
            m.blk_sl->resident = m.resident && gcn_direct;  // (fast precision only)
            // (synchronises s: host[0] and host[1] are current after the call)
            m.blk_sl->after_split = m.fork_hook;
            const bool built =
                build_blocked_self_loops(*m.blk_sl, n, nnz, rp, ci, r_unit, maxf, s, chunk);
            if (unit_late) {
                unit_v = host[0] == 1;
                m.unit_guess = unit_v;
            }
            if (built && host[1] == 0 && (unit_v || !gcn_direct)) {
                m.blk_sl->group_cols = gcn_direct ? 32 : 64;
                m.blk_sl_direct = true;
                m.unit_sl = gcn_direct;
            }
        }
        if (!m.blk_sl_direct) {
            m.sl_rp.reserve((n + 1) * sizeof(int32_t));
            m.sl_ci.reserve((nnz + n) * sizeof(int32_t));
            m.sl_v.reserve((nnz + n) * sizeof(float));
            m.sl_values = m.need_norm() && !(unit_v && will_block);
            if (m.need_norm()) {
                m.dis.reserve(n * sizeof(float));
                gcn_norm(n, nnz, rp, ci, v, m.sl_rp.as<int32_t>(), m.sl_ci.as<int32_t>(),
                         m.sl_v.as<float>(), nullptr, m.dis.as<float>(), m.work.get(),
                         m.work.size(), s, m.sl_values);
            } else {
                add_self_loops(n, nnz, rp, ci, v, m.sl_rp.as<int32_t>(), m.sl_ci.as<int32_t>(),
                               m.sl_v.as<float>(), m.work.get(), m.work.size(), s, false);
            }
            if (unit_v) {
                // no diagonal in A: A + I has nnz + n entries
                TG_HIP(hipMemcpyAsync(host + 1, m.sl_rp.as<int32_t>() + n, sizeof(int32_t),
                                      hipMemcpyDeviceToHost, s));
                TG_HIP(hipStreamSynchronize(s));
                m.unit_sl = host[1] == nnz + n;
                if (!m.unit_sl && !m.sl_values) {  // a diagonal of A: A + I holds a 2
                    m.sl_values = true;
                    gcn_norm(n, nnz, rp, ci, v, m.sl_rp.as<int32_t>(), m.sl_ci.as<int32_t>(),
                             m.sl_v.as<float>(), nullptr, m.dis.as<float>(), m.work.get(),
                             m.work.size(), s, true);
                }
            }
        }
        // A + I's row plan is built by ensure_plan_sl, once the blocking is known
        if (!m.plan_sl) m.plan_sl = std::make_unique<tg_spmm_plan_s>();
        m.plan_sl_built = false;
    } else {
        m.plan_sl.reset();
    }
    m.have_cache = true;
    m.built_precision = m.precision;
    m.built_layers_gen = m.layers_gen;
    m.key_rp = rp;
    m.key_ci = ci;
    m.key_v = v;
    m.key_n = n;
    m.key_nnz = nnz;
    // column blocking in both modes: with the reference's per-call
    // preprocessing (config E) GCN / SAGE / GAT took 22.4 / 21.5 / 23.4 ms
    // unblocked and 14.8 / 12.0 / 17.3 ms blocked with everything rebuilt in
    // place (the block plans counted before one synchronisation)
    prepare_blocked(m, n, nnz, rp, ci, s);
    if (m.need_norm() || m.need_sl()) ensure_plan_sl(m, n, nnz, s);
    ensure_plan_raw(m, n, nnz, rp, s);
}

// GAT's scores buffer: src and dst scores [n x heads], then the blocked
// path's row statistics or softmax state [n x slots]
size_t scores_bytes(const tg_model_s& m, int64_t n) {
    int64_t heads_max = 1, slots_max = 1;
    for (auto& l : m.layers) {
        heads_max = std::max(heads_max, l.heads);
        if (l.type == LType::GAT) slots_max = std::max(slots_max, gat_stat_slots(l.heads, l.out));
    }
    return static_cast<size_t>(2 * heads_max + 2 * slots_max) * n * sizeof(float) + 256;
}

// Layer 0's transform beside the preprocessing: what it computed, in which
// layout.  The layout is the one the preprocessing most likely leads to
// (blocked where the default blocking applies; for GCN in fast precision, a
// unit A + I split from A directly: the factored aggregation); `matches`
// checks it against the preprocessing's outcome, and layer 0 recomputes
// the transform when it differs.
struct PreTransform {
    bool ready = false;     // planned: its buffers reserved, its layout chosen
    bool deferred = false;  // to start inside the preprocessing (a blocked build)
    bool on = false;        // launched
    bool tiled = false;     // GCN / SAGE: T tile-major
    bool factored = false;  // GCN: rows scaled by D^-1/2
};

// Chooses layer 0's side-stream transform and reserves its buffers (before
// any of the call's work is in flight).
PreTransform plan_pre_transform(tg_model_s& m, int64_t n, int64_t nnz) {
    PreTransform p;
    const Layer& l = m.layers[0];
    const bool exact = m.precision == TG_PRECISION_EXACT;
    const bool sage_tf =
        l.type == LType::SAGE &&
        sage_dataflow_for(exact ? TG_SAGE_CONCAT : m.sage_dataflow, l.agg, l.in, l.out, nnz) ==
            TG_SAGE_TRANSFORM_FIRST;
    if (l.type == LType::SAGE && !sage_tf) return p;  // (the aggregation comes first)
    if (!m.side) {
        TG_HIP(hipStreamCreateWithFlags(&m.side, hipStreamNonBlocking));
        TG_HIP(hipEventCreateWithFlags(&m.ev_fork, hipEventDisableTiming));
        TG_HIP(hipEventCreateWithFlags(&m.ev_join, hipEventDisableTiming));
    }
    // buffers first (a reallocation must not meet work in flight)
    if (l.type == LType::GCN) {
        const int gc = (!exact && !m.need_sl()) ? 32 : 64;
        p.tiled = resolve_block_rows(m.block_rows, n, nnz + n, gc) > 0;
        p.factored = p.tiled && !exact && !m.need_sl();
        m.pre.reserve(n * round_up(gather_pitch(l.out), 32) * sizeof(float));
        if (p.factored) {
            m.pre_dis.reserve(n * sizeof(float));
            m.pre_flag.reserve(sizeof(int32_t));
        }
    } else if (l.type == LType::GAT) {
        m.pre.reserve(n * gather_pitch(l.wide()) * sizeof(float));
        m.scores.reserve(scores_bytes(m, n));
    } else {
        p.tiled = sage_tf_tiled(l.out, l.agg == TG_AGG_MEAN &&
                                           resolve_block_rows(m.block_rows, n, nnz, 32) > 0);
        m.pre.reserve(sage_tf_floats(n, l.out) * sizeof(float));
        m.pre_w.reserve(l.in * 2 * gather_pitch(l.out) * sizeof(float));
    }
    // whether the preprocessing builds a blocked copy (A + I's in either
    // lane-group width, or A's for SAGE's mean) to start it from
    const bool sl_blk = (m.need_norm() || m.need_sl()) &&
                        (resolve_block_rows(m.block_rows, n, nnz + n, 32) > 0 ||
                         resolve_block_rows(m.block_rows, n, nnz + n, 64) > 0);
    const bool raw_blk = m.need_raw_mean() && resolve_block_rows(m.block_rows, n, nnz, 32) > 0;
    p.deferred = sl_blk || raw_blk;
    p.ready = true;
    return p;
}

// Launches layer 0's transform planned by plan_pre_transform on the side
// stream, after the work enqueued on s so far.
void fork_pre_transform(tg_model_s& m, PreTransform& p, int64_t n, const int32_t* rp,
                        const float* x, hipStream_t s) {
    if (!p.ready || p.on) return;
    const Layer& l = m.layers[0];
    const bool exact = m.precision == TG_PRECISION_EXACT;
    const int algo = exact ? TG_GEMM_INORDER : TG_GEMM_AUTO;
    hipStream_t t = m.side;
    TG_HIP(hipEventRecord(m.ev_fork, s));
    TG_HIP(hipStreamWaitEvent(t, m.ev_fork, 0));
    if (l.type == LType::GCN) {
        if (p.factored) {
            fill_i32(m.pre_flag.as<int32_t>(), 1, 0, t);
            unit_self_loop_dis(n, rp, m.pre_dis.as<float>(), m.pre_flag.as<int32_t>(), t);
        }
        GemmArgs g;
        g.m = n;
        g.n = l.out;
        g.a1 = x;
        g.lda1 = l.in;
        g.b1 = l.w.as<float>();
        g.ldb1 = l.out;
        g.k1 = l.in;
        g.c = m.pre.as<float>();
        g.ldc = p.tiled ? 32 : gather_pitch(l.out);
        g.c_tile_stride = p.tiled ? n * 32 : 0;
        if (p.factored) g.row_scale = m.pre_dis.as<float>();
        gemm(g, algo, t);
    } else if (l.type == LType::GAT) {
        const int64_t wide = l.wide(), ldwh = gather_pitch(wide);
        GemmArgs g;
        g.m = n;
        g.n = wide;
        g.a1 = x;
        g.lda1 = l.in;
        g.b1 = l.w.as<float>();
        g.ldb1 = wide;
        g.k1 = l.in;
        g.c = m.pre.as<float>();
        g.ldc = ldwh;
        gemm(g, algo, t);
        float* src = m.scores.as<float>();
        gat_scores(n, l.heads, l.out, m.pre.as<float>(), ldwh, l.al.as<float>(),
                   l.ar.as<float>(), src, src + n * l.heads, t);
    } else {
        sage_transform(n, l.in, l.out, x, l.wn.as<float>(), l.ws.as<float>(), p.tiled,
                       m.pre.as<float>(), m.pre_w.as<float>(), t, algo);
    }
    TG_HIP(hipEventRecord(m.ev_join, t));
    p.on = true;
}

// Whether the side stream's transform has the layout layer 0 needs after
// the preprocessing.
bool pre_matches(const tg_model_s& m, const PreTransform& p) {
    if (!p.on) return false;
    const Layer& l = m.layers[0];
    if (l.type == LType::GCN) {
        const bool tiled = m.blk_sl != nullptr;
        const bool factored = tiled && m.unit_sl;
        // (a factored transform's D^-1/2 is the one the direct split checked)
        return tiled == p.tiled && factored == p.factored && (!factored || m.blk_sl_direct);
    }
    if (l.type == LType::SAGE) return sage_tf_tiled(l.out, m.blk_raw != nullptr) == p.tiled;
    return true;
}

void forward(tg_model_s& m, int64_t n, int64_t nnz, const int32_t* rp, const int32_t* ci,
             const float* v, int64_t f_in, const float* x, float* out, int mode, hipStream_t s) {
    if (m.layers.empty()) throw std::runtime_error("Model::forward: no layers configured.");
    require(mode == TG_FORWARD_REFERENCE || mode == TG_FORWARD_CACHED,
            "Model::forward: unknown mode");
    require(n >= 0 && nnz >= 0 && f_in >= 0, "Model::forward: negative size");
    require(n < (int64_t(1) << 31) && nnz < (int64_t(1) << 31),
            "Model::forward: sizes must be < 2^31 (int32 CSR)");
    // the first layer's own shape check (layers.cpp:302-306, :551-555, :964-968)
    {
        const Layer& l0 = m.layers[0];
        const char* name = l0.type == LType::GCN ? "GCNLayer" : l0.type == LType::SAGE
                                                                 ? "SAGELayer" : "GATLayer";
        if (f_in != l0.in)
            throw std::invalid_argument(std::string(name) + "::forward: H has " +
                                        std::to_string(f_in) +
                                        " columns but layer expects in_features=" +
                                        std::to_string(l0.in) + ".");
    }
    for (size_t li = 1; li < m.layers.size(); ++li)
        if (m.layers[li].in != m.layers[li - 1].out_cols())
            throw std::invalid_argument("Model::forward: layer " + std::to_string(li) +
                                        " expects in_features=" +
                                        std::to_string(m.layers[li].in) + " but layer " +
                                        std::to_string(li - 1) + " produces " +
                                        std::to_string(m.layers[li - 1].out_cols()) + ".");
    if (n == 0) return;
    require(rp && x && out, "Model::forward: null pointer");
    require(nnz == 0 || (ci && v), "Model::forward: null pointer");

    // a reference-semantics call preprocesses the adjacency every time:
    // layer 0's transform runs beside it on the side stream (a cached call's
    // one-time build keeps the single stream, and allocates no side buffers)
    // It starts when the preprocessing's first blocked build has enqueued
    // its scatter: the split's passes are latency-bound and slow down several
    // times beside the GEMM, whose workgroups hold the CUs' slots; without a
    // blocked build it starts at once.
    PreTransform pre;
    if (mode == TG_FORWARD_REFERENCE && !adjacency_cached(m, n, nnz, rp, ci, v, mode))
        pre = plan_pre_transform(m, n, nnz);
    auto clear_hooks = [&]() {
        m.fork_hook = nullptr;
        if (m.blk_sl) m.blk_sl->after_split = nullptr;
        if (m.blk_raw) m.blk_raw->after_split = nullptr;
    };
    clear_hooks();
    if (pre.ready && pre.deferred)
        m.fork_hook = [&m, &pre, n, rp, x, s]() { fork_pre_transform(m, pre, n, rp, x, s); };
    else
        fork_pre_transform(m, pre, n, rp, x, s);
    try {
        prepare_adjacency(m, n, nnz, rp, ci, v, mode, s);
    } catch (...) {
        clear_hooks();
        throw;
    }
    clear_hooks();
    fork_pre_transform(m, pre, n, rp, x, s);  // (no blocked build started it)
    if (pre.on) TG_HIP(hipStreamWaitEvent(s, m.ev_join, 0));
    const bool use_pre = pre_matches(m, pre);

    // precision: the exact mode keeps the reference's operation order
    const bool exact = m.precision == TG_PRECISION_EXACT;
    const int algo = exact ? TG_GEMM_INORDER : TG_GEMM_AUTO;
    const int dataflow = exact ? TG_SAGE_CONCAT : m.sage_dataflow;

    // buffers
    const int64_t wmax = m.max_wide();
    size_t ws = 0;
    for (auto& l : m.layers) {
        if (l.type == LType::SAGE)
            ws = std::max(ws, sage_forward_ws(n, l.in, l.out, l.agg, dataflow, nnz));
        if (l.type == LType::GAT)
            ws = std::max(ws, m.blk_sl_direct
                                  ? gat_workspace_blocked(*m.blk_sl, n, l.heads, l.out, l.concat)
                                  : gat_workspace(*m.plan_sl, n, l.heads, l.out, l.concat));
    }
    m.act[0].reserve(n * wmax * sizeof(float));
    m.act[1].reserve(n * wmax * sizeof(float));
    // the transform's output: row-major at gather_pitch, or tile-major (32-column
    // tiles of n rows) for the blocked aggregations
    m.tmp.reserve(n * round_up(gather_pitch(wmax), 32) * sizeof(float));
    m.scores.reserve(scores_bytes(m, n));
    m.work.reserve(ws);

    const float* h = x;
    for (size_t li = 0; li < m.layers.size(); ++li) {
        const Layer& l = m.layers[li];
        const bool last = li + 1 == m.layers.size();
        float* y = last ? out : m.act[li % 2].as<float>();
        if (l.type == LType::GCN) {
            // H*W, then A_norm * (H*W) + b -> act -> post  (layers.cpp:319-336);
            // H*W's rows are padded (gather_pitch) for 128-bit, line-aligned gathers
            // (blocked: tile-major, each 32-column tile one slab of n rows)
            const bool tiled = m.blk_sl != nullptr;
            // factored (unit A + I, blocked): D^-1/2 in the GEMM's and the
            // aggregation's stores, an unweighted blocked copy
            const bool factored = tiled && m.unit_sl;
            const int64_t ldhw = tiled ? 32 : gather_pitch(l.out);
            // (layer 0: computed beside the preprocessing, same layout)
            float* hw = li == 0 && use_pre ? m.pre.as<float>() : m.tmp.as<float>();
            if (!(li == 0 && use_pre)) {
                GemmArgs g;
                g.m = n;
                g.n = l.out;
                g.a1 = h;
                g.lda1 = l.in;
                g.b1 = l.w.as<float>();
                g.ldb1 = l.out;
                g.k1 = l.in;
                g.c = hw;
                g.ldc = ldhw;
                g.c_tile_stride = tiled ? n * 32 : 0;
                if (factored) g.row_scale = m.dis.as<float>();
                gemm(g, algo, s);
            }
            AggEpilogue epi;
            if (factored) {
                epi.row_scale = m.dis.as<float>();
                epi.scale_ld = 1;
                epi.scale_cols = static_cast<int>(l.out);
                epi.mask_tail = 1;
            }
            epi.bias = l.bias ? l.b.as<float>() : nullptr;
            epi.act = l.act;
            epi.post = l.post;
            epi.b_tile_stride = tiled ? n * 32 : 0;
            if (tiled)
                run_aggregate_blocked(*m.blk_sl, l.out, hw, ldhw, y, l.out, epi, s);
            else
                run_aggregate(*m.plan_sl, l.out, m.sl_ci.as<int32_t>(), m.sl_v.as<float>(), hw,
                              ldhw, y, l.out, epi, s);
        } else if (l.type == LType::SAGE) {
            sage_forward(*m.plan_raw, n, l.in, l.out, l.agg, ci, h, l.wn.as<float>(),
                         l.ws.as<float>(), l.bias ? l.b.as<float>() : nullptr, l.act, l.post,
                         dataflow, y, m.work.get(), m.work.size(), s, algo,
                         l.agg == TG_AGG_MEAN ? m.blk_raw.get() : nullptr,
                         li == 0 && use_pre ? m.pre.as<float>() : nullptr);
        } else {
            const int64_t wide = l.heads * l.out;
            // line-aligned rows for the gathers (row-major: the score kernel
            // reads each row's heads; a tile-major Wh measured 0.3 ms slower)
            const bool blocked = m.blk_sl != nullptr && gat_blocked_ok(l.heads, l.out, l.concat);
            const int64_t ldwh = gather_pitch(wide);
            // (layer 0: computed beside the preprocessing, scores included)
            float* wh = li == 0 && use_pre ? m.pre.as<float>() : m.tmp.as<float>();
            float* src = m.scores.as<float>();
            float* dst = src + n * l.heads;
            if (!(li == 0 && use_pre)) {
                GemmArgs g;
                g.m = n;
                g.n = wide;
                g.a1 = h;
                g.lda1 = l.in;
                g.b1 = l.w.as<float>();
                g.ldb1 = wide;
                g.k1 = l.in;
                g.c = wh;
                g.ldc = ldwh;
                gemm(g, algo, s);
                gat_scores(n, l.heads, l.out, wh, ldwh, l.al.as<float>(), l.ar.as<float>(), src,
                           dst, s);
            }
            if (blocked) {
                float* rmax = dst + n * l.heads;
                float* rinv = rmax + n * gat_stat_slots(l.heads, l.out);
                gat_aggregate_blocked(*m.blk_sl, m.blk_sl_direct ? nullptr : m.plan_sl.get(), n,
                                      l.heads, l.out,
                                      m.sl_ci.as<int32_t>(), wh, ldwh, src, dst, l.slope,
                                      l.bias ? l.b.as<float>() : nullptr, l.act, l.post, y,
                                      l.out_cols(), rmax, rinv, m.work.get(), m.work.size(), s,
                                      exact, l.ar.as<float>());
            } else {
                gat_aggregate(*m.plan_sl, n, l.heads, l.out, m.sl_ci.as<int32_t>(), wh, ldwh,
                              src, dst, l.slope, l.bias ? l.b.as<float>() : nullptr, l.act,
                              l.post, l.concat, y, l.out_cols(), m.work.get(), m.work.size(), s,
                              exact);
            }
        }
        h = y;
    }
}

}  // namespace
}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_model_create(tg_model_t* model_out) {
    return guard([&] {
        require(model_out != nullptr, "tg_model_create: model_out is null");
        *model_out = new tg_model_s();
    });
}

int tg_model_destroy(tg_model_t model) {
    return guard([&] { delete model; });
}

int tg_model_add_gcn_layer(tg_model_t model, int64_t in_f, int64_t out_f, int bias, int act,
                           int post, int64_t* index_out) {
    return guard([&] {
        require(model != nullptr, "model is null");
        Layer l;
        l.type = LType::GCN;
        l.in = in_f;
        l.out = out_f;
        l.bias = bias != 0;
        l.act = act;
        l.post = post;
        const int64_t i = tg::add_layer(*model, std::move(l));
        if (index_out) *index_out = i;
    });
}

int tg_model_add_sage_layer(tg_model_t model, int64_t in_f, int64_t out_f, int agg, int bias,
                            int act, int post, int64_t* index_out) {
    return guard([&] {
        require(model != nullptr, "model is null");
        Layer l;
        l.type = LType::SAGE;
        l.in = in_f;
        l.out = out_f;
        l.agg = agg;
        l.bias = bias != 0;
        l.act = act;
        l.post = post;
        const int64_t i = tg::add_layer(*model, std::move(l));
        if (index_out) *index_out = i;
    });
}

int tg_model_add_gat_layer(tg_model_t model, int64_t in_f, int64_t out_f, int64_t heads,
                           int concat, float neg_slope, int bias, int act, int post,
                           int64_t* index_out) {
    return guard([&] {
        require(model != nullptr, "model is null");
        Layer l;
        l.type = LType::GAT;
        l.in = in_f;
        l.out = out_f;
        l.heads = heads;
        l.concat = concat != 0;
        l.slope = neg_slope;
        l.bias = bias != 0;
        l.act = act;
        l.post = post;
        const int64_t i = tg::add_layer(*model, std::move(l));
        if (index_out) *index_out = i;
    });
}

int tg_model_num_layers(tg_model_t model, int64_t* n_out) {
    return guard([&] {
        require(model != nullptr && n_out != nullptr, "null argument");
        *n_out = static_cast<int64_t>(model->layers.size());
    });
}

int tg_model_output_cols(tg_model_t model, int64_t* cols_out) {
    return guard([&] {
        require(model != nullptr && cols_out != nullptr, "null argument");
        if (model->layers.empty()) throw std::runtime_error("Model::forward: no layers configured.");
        *cols_out = model->layers.back().out_cols();
    });
}

int tg_model_set_tensor(tg_model_t model, const char* name, int64_t rows, int64_t cols,
                        const float* host_data) {
    return guard([&] {
        require(model != nullptr && name != nullptr, "null argument");
        require(rows >= 0 && cols >= 0, "tg_model_set_tensor: negative shape");
        require(rows * cols == 0 || host_data != nullptr, "tg_model_set_tensor: data is null");
        HostTensor t;
        t.rows = rows;
        t.cols = cols;
        t.data.assign(host_data, host_data + rows * cols);
        model->staged[name] = std::move(t);
    });
}

int tg_model_set_precision(tg_model_t model, int precision) {
    return guard([&] {
        require(model != nullptr, "model is null");
        require(precision == TG_PRECISION_FAST || precision == TG_PRECISION_EXACT,
                "unknown precision");
        model->precision = precision;
    });
}

int tg_model_set_blocking(tg_model_t model, int64_t rows_per_block) {
    return guard([&] {
        require(model != nullptr, "model is null");
        require(rows_per_block >= -1, "tg_model_set_blocking: rows_per_block must be >= -1");
        model->block_rows = rows_per_block;
    });
}

int tg_model_blocking_info(tg_model_t model, int64_t* blocks_sl, int64_t* cols_sl,
                           int64_t* blocks_raw, int64_t* cols_raw, int64_t* sl_direct,
                           int64_t* resident) {
    return guard([&] {
        require(model != nullptr, "model is null");
        const tg::BlockedCSR* sl = model->have_cache ? model->blk_sl.get() : nullptr;
        const tg::BlockedCSR* raw = model->have_cache ? model->blk_raw.get() : nullptr;
        if (blocks_sl) *blocks_sl = sl ? sl->n_blocks : 0;
        if (cols_sl) *cols_sl = sl ? sl->group_cols : 0;
        if (blocks_raw) *blocks_raw = raw ? raw->n_blocks : 0;
        if (cols_raw) *cols_raw = raw ? raw->group_cols : 0;
        if (sl_direct) *sl_direct = sl && model->blk_sl_direct ? 1 : 0;
        auto res = [](const tg::BlockedCSR* b) { return b && b->resident_wgs > 0; };
        if (resident) *resident = (res(sl) ? 1 : 0) | (res(raw) ? 2 : 0);
    });
}

int tg_model_set_self_loop_split(tg_model_t model, int direct) {
    return guard([&] {
        require(model != nullptr, "model is null");
        model->direct_split = direct != 0;
        model->have_cache = false;
    });
}

int tg_model_set_resident_passes(tg_model_t model, int on) {
    return guard([&] {
        require(model != nullptr, "model is null");
        model->resident = on != 0;
        model->have_cache = false;
    });
}

int tg_model_invalidate(tg_model_t model) {
    return guard([&] {
        require(model != nullptr, "model is null");
        model->have_cache = false;
    });
}

int tg_model_clear_tensors(tg_model_t model) {
    return guard([&] {
        require(model != nullptr, "model is null");
        model->staged.clear();
    });
}

int tg_model_load_weights(tg_model_t model) {
    return guard([&] {
        require(model != nullptr, "model is null");
        tg::load_weights(*model);
    });
}

int tg_model_set_sage_dataflow(tg_model_t model, int dataflow) {
    return guard([&] {
        require(model != nullptr, "model is null");
        require(dataflow >= TG_SAGE_AUTO && dataflow <= TG_SAGE_TRANSFORM_FIRST,
                "unknown SAGE dataflow");
        model->sage_dataflow = dataflow;
    });
}

int tg_model_forward(tg_model_t model, int64_t n, int64_t nnz, const int32_t* row_ptr,
                     const int32_t* col_ind, const float* val, int64_t f_in, const float* x,
                     float* out, int mode, tg_stream_t stream) {
    return guard([&] {
        require(model != nullptr, "model is null");
        tg::forward(*model, n, nnz, row_ptr, col_ind, val, f_in, x, out, mode,
                    static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
