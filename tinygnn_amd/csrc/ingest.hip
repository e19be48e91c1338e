// ingest.hip -- TinyGNN's CSV graph ingestion on gfx950 (replaces
// GraphLoader::parse_edges and GraphLoader::parse_features, reference
// src/graph_loader.cpp:61-206, and the file reading of GraphLoader::load,
// :286-326).
//
// Pipeline, all on the device after the file read:
//   1. The file is read into HBM through two pinned staging buffers, so the
//      reads overlap the copies.
//   2. Line index.  Newline positions are compacted: each 16 KB tile counts
//      its '\n' bytes with 128-bit loads, the counts are scanned, and the
//      tiles write the positions.  Each newline-delimited segment is trimmed
//      of " \t\r\n" (read_lines, :38-53), and the non-empty ones are
//      compacted into [LB, LE) byte ranges.  Line i of the index is line i of
//      the reference's `lines` vector, so messages carry the same numbers
//      (i + 1).
//   3. The header test (is_header, :24-33) on line 0.
//   4. Edges: one thread per line, the first comma, then std::stoi of both
//      sides (:73-99).
//   5. Features: one wavefront per line.
//      * Pass A counts the fields (std::getline semantics: a trailing comma
//        yields no last field) and parses node_id.
//      * The last line of every node_id is marked; earlier ones are
//        overwritten in the reference (:191-197).
//      * Pass B finds the commas 1 KB at a time (16 B per lane; positions
//        compacted in LDS), and each lane converts whole fields with
//        std::stof's semantics (numparse.hpp), writing the marked lines' rows.
//
// Errors: every line computes its own error code.  An atomic minimum over
// (line << 3 | code) selects the first, which is the one the reference's
// sequential loop throws.  The host then formats the reference's message
// from that line's bytes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"
#include "device_utils.hpp"
#include "numparse.hpp"
#include "numparse_table.hpp"

namespace {

struct CsvMeta {
    unsigned long long first_err;  // (line << 3) | code; ~0 when none
    unsigned long long total_nl;   // newline count
    int32_t max_id;                // largest endpoint / node_id, -1 if none
    int32_t header;
};

}  // namespace

struct tg_csv_s {
    tg::DeviceBuffer own_text;  // the file's bytes, when tg_csv_open read it
    const unsigned char* text = nullptr;
    int64_t n_bytes = 0;
    std::string name;
    int64_t n_lines = 0;
    int header = 0;
    tg::DeviceBuffer lb, le;  // int64 [n_lines]
    tg::DeviceBuffer meta;    // CsvMeta
    tg::DeviceBuffer pow10;   // numparse::Pow10Entry [kPow10Count]
    // feature pass A, kept between tg_csv_feature_shape and the parse
    tg::DeviceBuffer node, cnt, tok;  // int32 [n_data]
    bool shape_done = false;
    int64_t rows = 0, cols = 0;
};

namespace tg {
namespace {

namespace np = numparse;

constexpr int kIdxBlock = 256;
constexpr int kIdxRounds = 4;
constexpr int64_t kIdxTileGranules = int64_t(kIdxBlock) * kIdxRounds;  // 16 KB

enum : int {
    kErrNone = 0,
    // edges
    kErrMalformed = 1,
    kErrInvalidInt = 2,
    kErrNegative = 3,
    // features
    kErrInvalidNode = 1,
    kErrNegativeNode = 2,
    kErrInvalidFeature = 3,
    kErrNoFeatures = 4,
    kErrInconsistent = 5,
};

__device__ __forceinline__ bool is_trim(unsigned c) {
    return c == ' ' || c == '\t' || c == '\r' || c == '\n';
}

// 4-bit mask of the bytes of w equal to the byte replicated in pat.
__device__ __forceinline__ uint32_t eq4(uint32_t w, uint32_t pat) {
    const uint32_t x = w ^ pat;
    const uint32_t y = ~(((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x | 0x7f7f7f7fu);
    return ((y >> 7) & 1u) | ((y >> 14) & 2u) | ((y >> 21) & 4u) | ((y >> 28) & 8u);
}
__device__ __forceinline__ uint32_t eq16(uint4 v, uint32_t pat) {
    return eq4(v.x, pat) | (eq4(v.y, pat) << 4) | (eq4(v.z, pat) << 8) | (eq4(v.w, pat) << 12);
}
// Bytes [lo, hi) of a 16-byte granule as a mask; lo <= hi within [0, 16].
__device__ __forceinline__ uint32_t range16(int64_t lo, int64_t hi) {
    lo = lo < 0 ? 0 : (lo > 16 ? 16 : lo);
    hi = hi < 0 ? 0 : (hi > 16 ? 16 : hi);
    if (hi <= lo) return 0u;
    return ((1u << hi) - 1u) & ~((1u << lo) - 1u);
}

// Granule g covers absolute addresses [a0 + 16 g, a0 + 16 g + 16); its bytes
// have text offsets 16 g - head + j.  Only granules holding at least one byte
// of the text are loaded (page-granular protection makes the rest of such a
// granule readable).
struct Granules {
    const uint4* a0;
    int64_t head;  // text - a0, in [0, 16)
    int64_t n;     // text bytes
    int64_t count;
    __device__ __forceinline__ uint32_t valid(int64_t g) const {
        const int64_t off = 16 * g - head;
        return range16(-off, n - off);
    }
};

Granules granules_of(const unsigned char* text, int64_t n) {
    Granules gr;
    const uintptr_t a = reinterpret_cast<uintptr_t>(text);
    gr.a0 = reinterpret_cast<const uint4*>(a & ~uintptr_t(15));
    gr.head = int64_t(a & 15);
    gr.n = n;
    gr.count = ceil_div(gr.head + n, 16);
    return gr;
}

__global__ void meta_init_kernel(CsvMeta* m) {
    m->first_err = ~0ull;
    m->total_nl = 0;
    m->max_id = -1;
    m->header = 0;
}

__global__ __launch_bounds__(kIdxBlock) void nl_count_kernel(Granules gr, int32_t* counts,
                                                             CsvMeta* meta) {
    __shared__ int32_t red[kIdxBlock / kWave];
    int c = 0;
    for (int r = 0; r < kIdxRounds; ++r) {
        const int64_t g = int64_t(blockIdx.x) * kIdxTileGranules + r * kIdxBlock + threadIdx.x;
        if (g < gr.count) c += __popc(eq16(gr.a0[g], 0x0a0a0a0au) & gr.valid(g));
    }
    c = wave_sum(c);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int w = 0; w < kIdxBlock / kWave; ++w) t += red[w];
        counts[blockIdx.x] = t;
        if (t) atomicAdd(&meta->total_nl, static_cast<unsigned long long>(t));
    }
}

__global__ __launch_bounds__(kIdxBlock) void nl_write_kernel(Granules gr, const int32_t* offs,
                                                             int64_t* nl) {
    __shared__ int32_t lds[kIdxBlock / kWave];
    int64_t base = offs[blockIdx.x];
    for (int r = 0; r < kIdxRounds; ++r) {
        const int64_t g = int64_t(blockIdx.x) * kIdxTileGranules + r * kIdxBlock + threadIdx.x;
        uint32_t m = 0;
        if (g < gr.count) m = eq16(gr.a0[g], 0x0a0a0a0au) & gr.valid(g);
        int32_t total;
        const int32_t ex = block_exclusive_scan<kIdxBlock>(int32_t(__popc(m)), lds, &total);
        int64_t pos = base + ex;
        while (m) {
            const int j = __ffs(m) - 1;
            m &= m - 1;
            nl[pos++] = 16 * g - gr.head + j;
        }
        base += total;
    }
}

__device__ __forceinline__ void segment_bounds(const unsigned char* text, int64_t n,
                                               const int64_t* nl, int64_t n_nl, int64_t k,
                                               int64_t* b_out, int64_t* e_out) {
    int64_t b = k ? nl[k - 1] + 1 : 0;
    int64_t e = k < n_nl ? nl[k] : n;
    while (b < e && is_trim(text[b])) ++b;
    while (e > b && is_trim(text[e - 1])) --e;
    *b_out = b;
    *e_out = e;
}

__global__ __launch_bounds__(256) void seg_flag_kernel(const unsigned char* text, int64_t n,
                                                       const int64_t* nl, int64_t n_nl,
                                                       int32_t* flags) {
    const int64_t k = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k > n_nl) return;
    int64_t b, e;
    segment_bounds(text, n, nl, n_nl, k, &b, &e);
    flags[k] = b < e ? 1 : 0;
}

__global__ __launch_bounds__(256) void seg_write_kernel(const unsigned char* text, int64_t n,
                                                        const int64_t* nl, int64_t n_nl,
                                                        const int32_t* pos, int64_t* lb,
                                                        int64_t* le) {
    const int64_t k = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k > n_nl) return;
    if (pos[k + 1] == pos[k]) return;  // empty after trimming
    int64_t b, e;
    segment_bounds(text, n, nl, n_nl, k, &b, &e);
    lb[pos[k]] = b;
    le[pos[k]] = e;
}

// is_header (graph_loader.cpp:24-33) on line 0: a letter or '_' before the
// first ',', ' ' or '\t'.
__global__ void header_kernel(const unsigned char* text, const int64_t* lb, const int64_t* le,
                              const int32_t* n_lines, CsvMeta* meta) {
    int h = 0;
    if (*n_lines > 0) {
        for (int64_t p = lb[0]; p < le[0]; ++p) {
            const unsigned c = text[p];
            if (c == ',' || c == ' ' || c == '\t') break;
            if (np::is_alpha(c) || c == '_') {
                h = 1;
                break;
            }
        }
    }
    meta->header = h;
}

__device__ __forceinline__ void record_error(CsvMeta* meta, int64_t line, int code) {
    atomicMin(&meta->first_err, (static_cast<unsigned long long>(line) << 3) | unsigned(code));
}

__device__ __forceinline__ void block_max_id(int v, CsvMeta* meta) {
    // one atomic per wavefront
    v = max(v, __shfl_xor(v, 32, kWave));
    v = max(v, __shfl_xor(v, 16, kWave));
    v = max(v, __shfl_xor(v, 8, kWave));
    v = max(v, __shfl_xor(v, 4, kWave));
    v = max(v, __shfl_xor(v, 2, kWave));
    v = max(v, __shfl_xor(v, 1, kWave));
    if ((threadIdx.x & (kWave - 1)) == 0 && v >= 0) atomicMax(&meta->max_id, v);
}

// GraphLoader::parse_edges (graph_loader.cpp:61-107), one thread per line.
__global__ __launch_bounds__(256) void edges_kernel(const unsigned char* text, const int64_t* lb,
                                                    const int64_t* le, int64_t start,
                                                    int64_t n_data, int32_t* src, int32_t* dst,
                                                    CsvMeta* meta) {
    const int64_t d = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    int best = -1;
    if (d < n_data) {
        const int64_t i = start + d;
        const int64_t b = lb[i], e = le[i];
        int64_t c = b;
        while (c < e && text[c] != ',') ++c;
        int32_t s = 0, t = 0;
        int err = kErrNone;
        if (c == e) {
            err = kErrMalformed;
        } else {
            const int r1 = np::parse_int(text + b, text + c, &s);
            const int r2 = np::parse_int(text + c + 1, text + e, &t);
            if (r1 != np::kOk || r2 != np::kOk) err = kErrInvalidInt;
            else if (s < 0 || t < 0) err = kErrNegative;
        }
        src[d] = s;
        dst[d] = t;
        if (err) record_error(meta, i, err);
        else best = max(s, t);
    }
    block_max_id(best, meta);
}

// Feature pass A (graph_loader.cpp:118-170): one wavefront per line counts
// the fields and parses node_id.  node[d] = node_id, or -1 (invalid) / -2
// (negative); cnt[d] = number of feature fields.
__global__ __launch_bounds__(kWave) void feat_a_kernel(const unsigned char* text,
                                                       const int64_t* lb, const int64_t* le,
                                                       int64_t start, int32_t* node,
                                                       int32_t* cnt, CsvMeta* meta) {
    const int64_t d = blockIdx.x;
    const int64_t i = start + d;
    const int lane = threadIdx.x;
    const int64_t b = lb[i], e = le[i];
    const uintptr_t base = reinterpret_cast<uintptr_t>(text);
    const uintptr_t a_first = (base + b) & ~uintptr_t(15);
    const uintptr_t a_end = base + e;
    int commas = 0;
    for (uintptr_t a = a_first + 16 * lane; a < a_end; a += 16 * kWave) {
        const uint4 v = *reinterpret_cast<const uint4*>(a);
        const int64_t off = int64_t(a - base);
        commas += __popc(eq16(v, 0x2c2c2c2cu) & range16(b - off, e - off));
    }
    commas = wave_sum(commas);
    if (lane == 0) {
        const int fields = commas + 1 - (text[e - 1] == ',' ? 1 : 0);
        cnt[d] = fields - 1;
        int64_t c = b;
        while (c < e && text[c] != ',') ++c;
        int32_t id = 0;
        const int r = np::parse_int(text + b, text + c, &id);
        if (r != np::kOk) {
            node[d] = -1;
        } else if (id < 0) {
            node[d] = -2;
        } else {
            node[d] = id;
            atomicMax(&meta->max_id, id);
        }
    }
}

__global__ __launch_bounds__(256) void winner_kernel(const int32_t* node, int64_t n_data,
                                                     int32_t* winner) {
    const int64_t d = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (d >= n_data) return;
    const int32_t id = node[d];
    if (id >= 0) atomicMax(&winner[id], int32_t(d));
}

__global__ __launch_bounds__(256) void zero_rows_kernel(const int32_t* winner, int64_t rows,
                                                        int64_t n_rows, int64_t cols, int64_t ld,
                                                        float* out) {
    const int64_t n = n_rows * cols;
    for (int64_t k = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; k < n;
         k += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = k / cols;
        if (r >= rows || winner[r] < 0) out[r * ld + (k % cols)] = 0.0f;
    }
}

// Feature pass B (graph_loader.cpp:150-168,185-197), one wavefront per line.
constexpr int kWindow = 16 * kWave;  // bytes per step

__global__ __launch_bounds__(kWave) void feat_b_kernel(
    const unsigned char* text, const int64_t* lb, const int64_t* le, int64_t start,
    const int32_t* node, const int32_t* cnt, const int32_t* winner,
    const np::Pow10Entry* pow10, int64_t ld, float* out, int32_t* tok, CsvMeta* meta) {
    __shared__ int32_t cpos[kWindow];
    const int64_t d = blockIdx.x;
    const int64_t i = start + d;
    const int lane = threadIdx.x;
    const int64_t b = lb[i], e = le[i];
    const int32_t id = node[d];
    const int32_t my_cnt = cnt[d];
    const int32_t expected = cnt[0];
    const bool writable = id >= 0 && winner[id] == int32_t(d) && my_cnt == expected;
    const uintptr_t base = reinterpret_cast<uintptr_t>(text);
    const uintptr_t a_end = base + e;
    int64_t carry = b;     // start of the field in progress
    int64_t t0 = 0;        // index of the field ending at the window's first comma
    int bad = 0x7fffffff;  // first field that fails to convert
    auto convert = [&](int64_t fs, int64_t fe, int64_t t) {
        if (t < 1) return;  // field 0 is node_id (pass A)
        uint32_t bits;
        const int r = np::parse_float(text + fs, text + fe, pow10, &bits);
        if (r != np::kOk) {
            bad = min(bad, int(t));
        } else if (writable) {
            out[int64_t(id) * ld + (t - 1)] = __uint_as_float(bits);
        }
    };
    for (uintptr_t w = (base + b) & ~uintptr_t(15); w < a_end; w += kWindow) {
        const uintptr_t a = w + 16 * lane;
        uint32_t m = 0;
        if (a < a_end) {
            const uint4 v = *reinterpret_cast<const uint4*>(a);
            const int64_t off = int64_t(a - base);
            m = eq16(v, 0x2c2c2c2cu) & range16(b - off, e - off);
        }
        const int c = __popc(m);
        const int incl = wave_inclusive_scan(c);
        const int k_total = __shfl(incl, kWave - 1, kWave);
        int p = incl - c;
        while (m) {
            const int j = __ffs(m) - 1;
            m &= m - 1;
            cpos[p++] = int32_t(16 * lane + j);  // offset from w
        }
        __syncthreads();
        const int64_t wo = int64_t(w - base);
        for (int j = lane; j < k_total; j += kWave) {
            const int64_t fs = j == 0 ? carry : wo + cpos[j - 1] + 1;
            convert(fs, wo + cpos[j], t0 + j);
        }
        if (k_total > 0) carry = wo + cpos[k_total - 1] + 1;
        t0 += k_total;
        __syncthreads();
    }
    if (lane == 0 && carry < e) convert(carry, e, t0);  // the last field
    for (int s = kWave / 2; s > 0; s >>= 1) bad = min(bad, __shfl_xor(bad, s, kWave));
    if (lane == 0) {
        int err = kErrNone;
        if (id == -1) err = kErrInvalidNode;
        else if (id == -2) err = kErrNegativeNode;
        else if (bad != 0x7fffffff) err = kErrInvalidFeature;
        else if (d == 0 && my_cnt == 0) err = kErrNoFeatures;
        else if (my_cnt != expected) err = kErrInconsistent;
        if (err) {
            tok[d] = bad;
            record_error(meta, i, err);
        }
    }
}

// ---------------------------------------------------------------------------
// host side

const np::Pow10Entry* host_pow10() {
    static np::Pow10Entry tab[np::kPow10Count];
    static bool done = [] {
        np::build_pow10_table(tab);
        return true;
    }();
    (void)done;
    return tab;
}

CsvMeta read_meta(const tg_csv_s& c, hipStream_t s) {
    CsvMeta m;
    TG_HIP(hipMemcpyAsync(&m, c.meta.get(), sizeof m, hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    return m;
}

void reset_meta(tg_csv_s& c, hipStream_t s) {
    meta_init_kernel<<<1, 1, 0, s>>>(c.meta.as<CsvMeta>());
    TG_LAUNCH_CHECK();
}

unsigned grid_of(int64_t n, int block) { return static_cast<unsigned>(ceil_div(n, block)); }

void index_lines(tg_csv_s& c, hipStream_t s) {
    c.meta.resize(sizeof(CsvMeta));
    c.pow10.resize(sizeof(np::Pow10Entry) * np::kPow10Count);
    TG_HIP(hipMemcpyAsync(c.pow10.get(), host_pow10(), c.pow10.size(), hipMemcpyHostToDevice, s));
    reset_meta(c, s);
    c.n_lines = 0;
    c.header = 0;
    if (c.n_bytes == 0) {
        TG_HIP(hipStreamSynchronize(s));
        return;
    }
    const Granules gr = granules_of(c.text, c.n_bytes);
    const int64_t nb = ceil_div(gr.count, kIdxTileGranules);
    require(nb < (int64_t(1) << 31), "GraphLoader: file too large");
    DeviceBuffer counts(sizeof(int32_t) * nb), offs(sizeof(int32_t) * (nb + 1));
    DeviceBuffer temp(sizeof(int64_t) * scan_temp_elems(nb));
    nl_count_kernel<<<static_cast<unsigned>(nb), kIdxBlock, 0, s>>>(gr, counts.as<int32_t>(),
                                                                     c.meta.as<CsvMeta>());
    TG_LAUNCH_CHECK();
    const int64_t n_nl = int64_t(read_meta(c, s).total_nl);
    if (n_nl >= (int64_t(1) << 31) - 2)
        throw std::runtime_error("GraphLoader: more than 2^31 lines in '" + c.name + "'");
    exclusive_scan_i32(counts.as<int32_t>(), offs.as<int32_t>(), nb, temp.as<int64_t>(), s);
    DeviceBuffer nl(sizeof(int64_t) * std::max<int64_t>(n_nl, 1));
    nl_write_kernel<<<static_cast<unsigned>(nb), kIdxBlock, 0, s>>>(gr, offs.as<int32_t>(),
                                                                     nl.as<int64_t>());
    TG_LAUNCH_CHECK();
    const int64_t n_seg = n_nl + 1;
    DeviceBuffer flags(sizeof(int32_t) * n_seg), pos(sizeof(int32_t) * (n_seg + 1));
    DeviceBuffer temp2(sizeof(int64_t) * scan_temp_elems(n_seg));
    seg_flag_kernel<<<grid_of(n_seg, 256), 256, 0, s>>>(c.text, c.n_bytes, nl.as<int64_t>(), n_nl,
                                                        flags.as<int32_t>());
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(flags.as<int32_t>(), pos.as<int32_t>(), n_seg, temp2.as<int64_t>(), s);
    c.lb.resize(sizeof(int64_t) * n_seg);
    c.le.resize(sizeof(int64_t) * n_seg);
    seg_write_kernel<<<grid_of(n_seg, 256), 256, 0, s>>>(c.text, c.n_bytes, nl.as<int64_t>(), n_nl,
                                                         pos.as<int32_t>(), c.lb.as<int64_t>(),
                                                         c.le.as<int64_t>());
    TG_LAUNCH_CHECK();
    header_kernel<<<1, 1, 0, s>>>(c.text, c.lb.as<int64_t>(), c.le.as<int64_t>(),
                                  pos.as<int32_t>() + n_seg, c.meta.as<CsvMeta>());
    TG_LAUNCH_CHECK();
    int32_t n_lines = 0;
    TG_HIP(hipMemcpyAsync(&n_lines, pos.as<int32_t>() + n_seg, sizeof n_lines,
                          hipMemcpyDeviceToHost, s));
    const CsvMeta m = read_meta(c, s);  // synchronises (the buffers above die here)
    c.n_lines = n_lines;
    c.header = m.header;
}

// The trimmed text of line i (for messages).
std::string line_text(const tg_csv_s& c, int64_t i, hipStream_t s) {
    int64_t be[2];
    TG_HIP(hipMemcpyAsync(&be[0], c.lb.as<int64_t>() + i, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    TG_HIP(hipMemcpyAsync(&be[1], c.le.as<int64_t>() + i, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    std::string t(static_cast<size_t>(be[1] - be[0]), '\0');
    if (!t.empty())
        TG_HIP(hipMemcpy(&t[0], c.text + be[0], t.size(), hipMemcpyDeviceToHost));
    return t;
}

// Field k of a line split as std::getline(ss, token, ',') splits it.
std::string field_of(const std::string& line, int64_t k) {
    size_t b = 0;
    for (int64_t f = 0; f < k; ++f) {
        const size_t c = line.find(',', b);
        if (c == std::string::npos) return std::string();
        b = c + 1;
    }
    const size_t c = line.find(',', b);
    return line.substr(b, c == std::string::npos ? std::string::npos : c - b);
}

void read_file(const char* path, tg_csv_s& c, hipStream_t s) {
    const std::string p = path ? path : "";
    FILE* f = std::fopen(p.c_str(), "rb");
    if (!f) throw std::runtime_error("GraphLoader: cannot open file '" + p + "'");
    std::unique_ptr<FILE, int (*)(FILE*)> guard_f(f, std::fclose);
    if (std::fseek(f, 0, SEEK_END) != 0) throw std::runtime_error("GraphLoader: cannot read '" + p + "'");
    const int64_t n = static_cast<int64_t>(std::ftell(f));
    if (n < 0) throw std::runtime_error("GraphLoader: cannot read '" + p + "'");
    std::rewind(f);
    c.own_text.resize(static_cast<size_t>(std::max<int64_t>(n, 1)));
    constexpr size_t kStage = size_t(32) << 20;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    struct Cleanup {
        void** st;
        hipEvent_t* ev;
        ~Cleanup() {
            for (int k = 0; k < 2; ++k) {
                if (ev[k]) (void)hipEventSynchronize(ev[k]), (void)hipEventDestroy(ev[k]);
                if (st[k]) (void)hipHostFree(st[k]);
            }
        }
    } cleanup{stage, done};
    for (int k = 0; k < 2; ++k) {
        TG_HIP(hipHostMalloc(&stage[k], kStage, hipHostMallocDefault));
        TG_HIP(hipEventCreateWithFlags(&done[k], hipEventDisableTiming));
    }
    int64_t off = 0;
    for (int k = 0; off < n; k ^= 1) {
        TG_HIP(hipEventSynchronize(done[k]));  // the staging buffer is free again
        const size_t want = static_cast<size_t>(std::min<int64_t>(n - off, int64_t(kStage)));
        const size_t got = std::fread(stage[k], 1, want, f);
        if (got != want) throw std::runtime_error("GraphLoader: cannot read '" + p + "'");
        TG_HIP(hipMemcpyAsync(c.own_text.as<char>() + off, stage[k], got, hipMemcpyHostToDevice, s));
        TG_HIP(hipEventRecord(done[k], s));
        off += static_cast<int64_t>(got);
    }
    TG_HIP(hipStreamSynchronize(s));
    c.text = c.own_text.as<unsigned char>();
    c.n_bytes = n;
    c.name = p;
}

void feature_shape(tg_csv_s& c, hipStream_t s) {
    if (c.shape_done) return;
    if (c.n_lines == 0)
        throw std::runtime_error("GraphLoader::parse_features: file is empty: '" + c.name + "'");
    const int64_t n_data = c.n_lines - c.header;
    if (n_data == 0)
        throw std::runtime_error("GraphLoader::parse_features: no data rows in '" + c.name + "'");
    c.node.resize(sizeof(int32_t) * n_data);
    c.cnt.resize(sizeof(int32_t) * n_data);
    c.tok.resize(sizeof(int32_t) * n_data);
    reset_meta(c, s);
    feat_a_kernel<<<static_cast<unsigned>(n_data), kWave, 0, s>>>(
        c.text, c.lb.as<int64_t>(), c.le.as<int64_t>(), c.header, c.node.as<int32_t>(),
        c.cnt.as<int32_t>(), c.meta.as<CsvMeta>());
    TG_LAUNCH_CHECK();
    int32_t first_cnt = 0;
    TG_HIP(hipMemcpyAsync(&first_cnt, c.cnt.get(), sizeof first_cnt, hipMemcpyDeviceToHost, s));
    const CsvMeta m = read_meta(c, s);
    c.rows = int64_t(m.max_id) + 1;
    c.cols = std::max<int32_t>(first_cnt, 0);
    c.shape_done = true;
}

}  // namespace
}  // namespace tg

using tg::guard;
using tg::require;

extern "C" {

int tg_csv_open(const char* path, tg_csv_t* csv_out, tg_stream_t stream) {
    return guard([&] {
        require(csv_out != nullptr, "tg_csv_open: csv_out is null");
        *csv_out = nullptr;
        const auto s = static_cast<hipStream_t>(stream);
        auto c = std::make_unique<tg_csv_s>();
        tg::read_file(path, *c, s);
        tg::index_lines(*c, s);
        *csv_out = c.release();
    });
}

int tg_csv_index(const char* text, int64_t n_bytes, const char* name, tg_csv_t* csv_out,
                 tg_stream_t stream) {
    return guard([&] {
        require(csv_out != nullptr, "tg_csv_index: csv_out is null");
        *csv_out = nullptr;
        require(n_bytes >= 0, "tg_csv_index: negative size");
        require(n_bytes == 0 || text != nullptr, "tg_csv_index: text is null");
        auto c = std::make_unique<tg_csv_s>();
        c->text = reinterpret_cast<const unsigned char*>(text);
        c->n_bytes = n_bytes;
        c->name = name ? name : "";
        tg::index_lines(*c, static_cast<hipStream_t>(stream));
        *csv_out = c.release();
    });
}

int tg_csv_destroy(tg_csv_t csv) {
    return guard([&] {
        if (csv) TG_HIP(hipDeviceSynchronize());
        delete csv;
    });
}

int tg_csv_info(tg_csv_t csv, int64_t* n_lines, int* has_header) {
    return guard([&] {
        require(csv != nullptr, "tg_csv_info: csv is null");
        if (n_lines) *n_lines = csv->n_lines;
        if (has_header) *has_header = csv->header;
    });
}

int tg_csv_parse_edges(tg_csv_t csv, int32_t* src, int32_t* dst, int64_t* max_id_out,
                       tg_stream_t stream) {
    return guard([&] {
        require(csv != nullptr, "GraphLoader::parse_edges: csv is null");
        const auto s = static_cast<hipStream_t>(stream);
        if (csv->n_lines == 0)
            throw std::runtime_error("GraphLoader::parse_edges: file is empty: '" + csv->name +
                                     "'");
        const int64_t n_data = csv->n_lines - csv->header;
        require(n_data == 0 || (src && dst), "GraphLoader::parse_edges: null output");
        tg::reset_meta(*csv, s);
        if (n_data > 0) {
            tg::edges_kernel<<<tg::grid_of(n_data, 256), 256, 0, s>>>(
                csv->text, csv->lb.as<int64_t>(), csv->le.as<int64_t>(), csv->header, n_data,
                src, dst, csv->meta.as<CsvMeta>());
            TG_LAUNCH_CHECK();
        }
        const CsvMeta m = tg::read_meta(*csv, s);
        if (m.first_err != ~0ull) {
            const int64_t i = static_cast<int64_t>(m.first_err >> 3);
            const int code = static_cast<int>(m.first_err & 7u);
            const std::string ln = std::to_string(i + 1);
            if (code == tg::kErrNegative) {
                int32_t sd[2];
                TG_HIP(hipMemcpy(&sd[0], src + (i - csv->header), 4, hipMemcpyDeviceToHost));
                TG_HIP(hipMemcpy(&sd[1], dst + (i - csv->header), 4, hipMemcpyDeviceToHost));
                throw std::runtime_error("GraphLoader::parse_edges: negative node ID on line " +
                                         ln + ": src=" + std::to_string(sd[0]) +
                                         ", dst=" + std::to_string(sd[1]));
            }
            const std::string line = tg::line_text(*csv, i, s);
            if (code == tg::kErrMalformed)
                throw std::runtime_error("GraphLoader::parse_edges: malformed line " + ln + ": '" +
                                         line + "'");
            throw std::runtime_error("GraphLoader::parse_edges: invalid integer on line " + ln +
                                     ": '" + line + "'");
        }
        if (max_id_out) *max_id_out = m.max_id;
    });
}

int tg_csv_feature_shape(tg_csv_t csv, int64_t* rows, int64_t* cols, tg_stream_t stream) {
    return guard([&] {
        require(csv != nullptr, "GraphLoader::parse_features: csv is null");
        tg::feature_shape(*csv, static_cast<hipStream_t>(stream));
        if (rows) *rows = csv->rows;
        if (cols) *cols = csv->cols;
    });
}

int tg_csv_parse_features(tg_csv_t csv, float* out, int64_t n_rows, int64_t ld,
                          tg_stream_t stream) {
    return guard([&] {
        require(csv != nullptr, "GraphLoader::parse_features: csv is null");
        const auto s = static_cast<hipStream_t>(stream);
        tg::feature_shape(*csv, s);
        const int64_t rows = csv->rows, cols = csv->cols;
        require(n_rows >= rows, "GraphLoader::parse_features: n_rows below the table's rows");
        require(ld >= cols, "GraphLoader::parse_features: ld below the table's columns");
        require(out != nullptr || n_rows * cols == 0, "GraphLoader::parse_features: null output");
        const int64_t n_data = csv->n_lines - csv->header;
        tg::DeviceBuffer winner(sizeof(int32_t) * std::max<int64_t>(rows, 1));
        tg::fill_i32(winner.as<int32_t>(), rows, -1, s);
        tg::winner_kernel<<<tg::grid_of(n_data, 256), 256, 0, s>>>(csv->node.as<int32_t>(), n_data,
                                                                  winner.as<int32_t>());
        TG_LAUNCH_CHECK();
        if (n_rows * cols > 0) {
            const int64_t total = n_rows * cols;
            const unsigned g = static_cast<unsigned>(std::min<int64_t>(tg::ceil_div(total, 256), 65536));
            tg::zero_rows_kernel<<<g, 256, 0, s>>>(winner.as<int32_t>(), rows, n_rows, cols, ld, out);
            TG_LAUNCH_CHECK();
        }
        tg::reset_meta(*csv, s);
        tg::feat_b_kernel<<<static_cast<unsigned>(n_data), tg::kWave, 0, s>>>(
            csv->text, csv->lb.as<int64_t>(), csv->le.as<int64_t>(), csv->header,
            csv->node.as<int32_t>(), csv->cnt.as<int32_t>(), winner.as<int32_t>(),
            csv->pow10.as<tg::numparse::Pow10Entry>(), ld, out, csv->tok.as<int32_t>(),
            csv->meta.as<CsvMeta>());
        TG_LAUNCH_CHECK();
        const CsvMeta m = tg::read_meta(*csv, s);  // synchronises; winner dies after
        if (m.first_err == ~0ull) return;
        const int64_t i = static_cast<int64_t>(m.first_err >> 3);
        const int64_t d = i - csv->header;
        const int code = static_cast<int>(m.first_err & 7u);
        const std::string ln = std::to_string(i + 1);
        const std::string P = "GraphLoader::parse_features: ";
        if (code == tg::kErrNegativeNode) throw std::runtime_error(P + "negative node_id on line " + ln);
        if (code == tg::kErrNoFeatures) throw std::runtime_error(P + "no features on line " + ln);
        const std::string line = tg::line_text(*csv, i, s);
        if (code == tg::kErrInvalidNode)
            throw std::runtime_error(P + "invalid node_id on line " + ln + ": '" +
                                     tg::field_of(line, 0) + "'");
        if (code == tg::kErrInvalidFeature) {
            int32_t t = 0;
            TG_HIP(hipMemcpy(&t, csv->tok.as<int32_t>() + d, 4, hipMemcpyDeviceToHost));
            throw std::runtime_error(P + "invalid feature on line " + ln + ": '" +
                                     tg::field_of(line, t) + "'");
        }
        int32_t got = 0;
        TG_HIP(hipMemcpy(&got, csv->cnt.as<int32_t>() + d, 4, hipMemcpyDeviceToHost));
        throw std::runtime_error(P + "inconsistent feature count on line " + ln + ": expected " +
                                 std::to_string(cols) + " but got " + std::to_string(got));
    });
}

}  // extern "C"
