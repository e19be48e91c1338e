// graph.hip -- graph preprocessing on gfx950: CSR construction from an edge
// list, CSR validation, self-loop insertion and symmetric GCN normalisation.
//
// Every output here is bit-identical to the reference:
//   * edge_list_to_csr (reference src/graph_loader.cpp:211-281): row = src,
//     out-degree row_ptr, each row's destinations sorted ascending with
//     duplicates kept, values 1.0f.  The sorted multiset of a row is unique,
//     so the nondeterministic atomic scatter followed by a per-row sort
//     yields exactly the reference's bytes.
//   * add_self_loops (src/layers.cpp:71-144): existing diagonals become
//     v + 1.0f; a missing diagonal is inserted before the first column > i
//     in row order, or appended.
//   * gcn_norm (src/layers.cpp:158-208): deg = sequential fp32 sum over the
//     row of A+I, dis = 1/sqrt(deg) (correctly rounded), v' = (v*dis_i)*dis_j.
#include "common.hpp"
#include "device_utils.hpp"

#include <algorithm>
#include <climits>
#include <string>
#include <type_traits>
#include <vector>

namespace tg {
namespace {

constexpr int kSortWaveMax = 64;     // rows of 2..64 entries: one wave, registers
constexpr int kSortBlockMax = 1024;  // rows of 65..1024: 256 threads, LDS
constexpr int kSortBigMax = 16384;   // rows of 1025..16384: 1024 threads, 64 KB LDS
constexpr int kSortTile = 16384;     // longer rows: global bitonic, LDS tiles

__host__ __device__ inline int next_pow2(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// ---------------------------------------------------------------------------
// edge_list_to_csr
// ---------------------------------------------------------------------------

// Counts out-degrees of valid edges; records the first invalid endpoint as
// the key 2*edge + (0 = src, 1 = dst) (the reference checks src before dst,
// edges in order).
__global__ __launch_bounds__(256) void edge_count_kernel(const int32_t* __restrict__ src,
                                                         const int32_t* __restrict__ dst,
                                                         int64_t n_edges, int32_t n_nodes,
                                                         int check_dst,
                                                         int32_t* __restrict__ deg,
                                                         unsigned long long* __restrict__ bad) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n_edges;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int32_t s = src[e], d = dst[e];
        const bool sbad = s < 0 || s >= n_nodes;
        const bool dbad = check_dst && (d < 0 || d >= n_nodes);
        if (sbad || dbad) {
            atomicMin(bad, static_cast<unsigned long long>(2 * e + (sbad ? 0 : 1)));
        } else {
            atomicAdd(&deg[s], 1);
        }
    }
}

// Sorts rows into length classes: 0 = 2..64, 1 = 65..1024, 2 = 1025..16384,
// 3 = longer.  counts[c] ends as the class size.
// Positions are reserved per workgroup (LDS counts, one global atomic per
// class and workgroup), so the global counters see n/256 atomics, not n.
__global__ __launch_bounds__(256) void classify_rows_kernel(const int32_t* __restrict__ deg,
                                                            int64_t n,
                                                            int32_t* __restrict__ lists,
                                                            int32_t* __restrict__ counts) {
    __shared__ int lcount[4], lbase[4];
    if (threadIdx.x < 4) lcount[threadIdx.x] = 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int c = -1, lpos = 0;
    if (r < n) {
        const int d = deg[r];
        if (d >= 2) {
            c = d <= kSortWaveMax ? 0 : d <= kSortBlockMax ? 1 : d <= kSortBigMax ? 2 : 3;
            lpos = atomicAdd(&lcount[c], 1);
        }
    }
    __syncthreads();
    if (threadIdx.x < 4 && lcount[threadIdx.x] > 0)
        lbase[threadIdx.x] = atomicAdd(&counts[threadIdx.x], lcount[threadIdx.x]);
    __syncthreads();
    if (c >= 0) lists[static_cast<int64_t>(c) * n + lbase[c] + lpos] = static_cast<int32_t>(r);
}

__global__ __launch_bounds__(256) void edge_scatter_kernel(const int32_t* __restrict__ src,
                                                           const int32_t* __restrict__ dst,
                                                           int64_t n_edges,
                                                           const int32_t* __restrict__ row_ptr,
                                                           int32_t* __restrict__ cursor,
                                                           int32_t* __restrict__ col_ind,
                                                           float* __restrict__ val) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n_edges;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int32_t s = src[e];
        const int32_t pos = row_ptr[s] + atomicAdd(&cursor[s], 1);
        col_ind[pos] = dst[e];
        val[e] = 1.0f;
    }
}

// One wavefront sorts one row of 2..64 entries held one per lane.
__global__ __launch_bounds__(256) void sort_wave_kernel(const int32_t* __restrict__ rows,
                                                        int32_t n_rows,
                                                        const int32_t* __restrict__ row_ptr,
                                                        int32_t* __restrict__ col) {
    const int wid = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (wid >= n_rows) return;
    const int r = rows[wid];
    const int b = row_ptr[r];
    const int len = row_ptr[r + 1] - b;
    int x = lane < len ? col[b + lane] : INT_MAX;
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const int y = __shfl_xor(x, j, kWave);
            const bool up = (lane & k) == 0;
            const bool low = (lane & j) == 0;
            // lower index keeps the min on an ascending run, the max otherwise
            x = (low == up) ? min(x, y) : max(x, y);
        }
    }
    if (lane < len) col[b + lane] = x;
}

// Bitonic sort of n = 2^p keys in LDS by the whole workgroup; `dir_base` is
// the index of key 0 within the full sequence whose bitonic direction rule
// ((g & k) == 0 -> ascending) applies, and stages run for k in [k_lo, k_hi]
// and, within the first stage, j from j_hi down.
template <int BLOCK>
__device__ __forceinline__ void lds_bitonic(int* keys, int n, int64_t dir_base, int k_lo,
                                            int k_hi, int j_first) {
    for (int k = k_lo; k <= k_hi; k <<= 1) {
        for (int j = (k == k_lo ? j_first : (k >> 1)); j > 0; j >>= 1) {
            for (int p = threadIdx.x; p < (n >> 1); p += BLOCK) {
                const int i = ((p / j) * 2 * j) + (p % j);
                const int q = i + j;
                const bool up = ((dir_base + i) & k) == 0;
                const int a = keys[i], c = keys[q];
                if ((a > c) == up) {
                    keys[i] = c;
                    keys[q] = a;
                }
            }
            __syncthreads();
        }
    }
}

// One workgroup sorts one row of up to CAP entries in LDS.
template <int BLOCK, int CAP>
__global__ __launch_bounds__(BLOCK) void sort_block_kernel(const int32_t* __restrict__ rows,
                                                           const int32_t* __restrict__ row_ptr,
                                                           int32_t* __restrict__ col) {
    __shared__ int keys[CAP];
    const int r = rows[blockIdx.x];
    const int b = row_ptr[r];
    const int len = row_ptr[r + 1] - b;
    const int n = next_pow2(len);
    for (int t = threadIdx.x; t < n; t += BLOCK) keys[t] = t < len ? col[b + t] : INT_MAX;
    __syncthreads();
    lds_bitonic<BLOCK>(keys, n, 0, 2, n, 1);
    for (int t = threadIdx.x; t < len; t += BLOCK) col[b + t] = keys[t];
}

// Long rows: padded copies in a temp buffer of 16384-key tiles.  tile_off[t]
// is the offset (in keys) of tile t's row within the buffer, tile_len[t] the
// row's padded length.
__global__ __launch_bounds__(256) void long_gather_kernel(const int32_t* __restrict__ rows,
                                                          const int64_t* __restrict__ seg_off,
                                                          int32_t n_long,
                                                          const int32_t* __restrict__ row_ptr,
                                                          const int32_t* __restrict__ col,
                                                          int32_t* __restrict__ tmp) {
    const int lr = blockIdx.y;
    if (lr >= n_long) return;
    const int r = rows[lr];
    const int b = row_ptr[r];
    const int len = row_ptr[r + 1] - b;
    const int64_t off = seg_off[lr];
    const int64_t pad = seg_off[lr + 1] - off;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < pad;
         t += static_cast<int64_t>(gridDim.x) * 256)
        tmp[off + t] = t < len ? col[b + t] : INT_MAX;
}

__global__ __launch_bounds__(256) void long_scatter_kernel(const int32_t* __restrict__ rows,
                                                           const int64_t* __restrict__ seg_off,
                                                           int32_t n_long,
                                                           const int32_t* __restrict__ row_ptr,
                                                           int32_t* __restrict__ col,
                                                           const int32_t* __restrict__ tmp) {
    const int lr = blockIdx.y;
    if (lr >= n_long) return;
    const int r = rows[lr];
    const int b = row_ptr[r];
    const int len = row_ptr[r + 1] - b;
    const int64_t off = seg_off[lr];
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < len;
         t += static_cast<int64_t>(gridDim.x) * 256)
        col[b + t] = tmp[off + t];
}

// Tile-local bitonic stages (k in [k_lo, k_hi], j starting at j_first) on
// each 16384-key tile whose row is at least `min_pad` long.
__global__ __launch_bounds__(1024) void long_tile_kernel(int32_t* __restrict__ tmp,
                                                         const int64_t* __restrict__ tile_off,
                                                         const int64_t* __restrict__ tile_len,
                                                         int64_t min_pad, int k_lo, int k_hi,
                                                         int j_first) {
    __shared__ int keys[kSortTile];
    const int64_t t = blockIdx.x;
    if (tile_len[t] < min_pad) return;
    int32_t* base = tmp + t * kSortTile;
    const int64_t g0 = t * kSortTile - tile_off[t];  // index of key 0 within its row
    for (int i = threadIdx.x; i < kSortTile; i += 1024) keys[i] = base[i];
    __syncthreads();
    lds_bitonic<1024>(keys, kSortTile, g0, k_lo, k_hi, j_first);
    for (int i = threadIdx.x; i < kSortTile; i += 1024) base[i] = keys[i];
}

// One global compare-exchange step (stage k, distance j >= 16384) over all
// long rows whose padded length is >= k.
__global__ __launch_bounds__(256) void long_step_kernel(int32_t* __restrict__ tmp,
                                                        const int64_t* __restrict__ tile_off,
                                                        const int64_t* __restrict__ tile_len,
                                                        int64_t total, int64_t k, int64_t j) {
    for (int64_t x = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; x < total;
         x += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t t = x / kSortTile;
        if (tile_len[t] < k) continue;
        const int64_t g = x - tile_off[t];
        if (g & j) continue;  // the lower index of the pair does the exchange
        const int64_t y = x + j;
        const bool up = (g & k) == 0;
        const int32_t a = tmp[x], c = tmp[y];
        if ((a > c) == up) {
            tmp[x] = c;
            tmp[y] = a;
        }
    }
}

__global__ void write_i32_kernel(int32_t* p, int32_t v) { *p = v; }

// ---------------------------------------------------------------------------
// CSR validation (Tensor::sparse_csr checks, src/tensor.cpp:46-86)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void csr_check_kernel(const int32_t* __restrict__ row_ptr,
                                                        int64_t n_rows,
                                                        const int32_t* __restrict__ col_ind,
                                                        int64_t nnz, int64_t n_cols,
                                                        unsigned long long* __restrict__ bad) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (int64_t i = t0; i < nnz; i += stride) {
        const int32_t c = col_ind[i];
        if (c < 0 || c >= n_cols) atomicMin(&bad[0], static_cast<unsigned long long>(i));
    }
    for (int64_t i = t0 + 1; i <= n_rows; i += stride)
        if (row_ptr[i] < row_ptr[i - 1]) atomicMin(&bad[1], static_cast<unsigned long long>(i));
}

// ---------------------------------------------------------------------------
// Self-loops and normalisation
// ---------------------------------------------------------------------------
constexpr int kGroup = 16;      // lanes per row in the row-wise passes
constexpr int kLongRow = 2048;  // longer rows: one workgroup each (the *_long kernels)
constexpr int kLongBlock = 256;

// Correctly rounded (round-to-nearest) float sqrt and reciprocal for
// positive finite inputs, as the host's sqrtss / divss give them.  The
// device estimate is moved to the neighbouring float while the exact value
// lies outside its rounding interval; the midpoint tests are exact in
// double (a 25-bit midpoint squared, or times a 24-bit float, fits in 53
// bits), and neither sqrt(d) nor 1/s of a float can fall on a midpoint, so
// there are no ties.
__device__ __forceinline__ float next_up(float x) { return __int_as_float(__float_as_int(x) + 1); }
__device__ __forceinline__ float next_dn(float x) { return __int_as_float(__float_as_int(x) - 1); }

__device__ float cr_sqrt(float d) {
    float s = __fsqrt_rn(d);
    if (!(d > 0.0f) || !isfinite(d)) return s;
    const double dd = d;
    for (int it = 0; it < 4; ++it) {
        const double hi = 0.5 * (static_cast<double>(s) + static_cast<double>(next_up(s)));
        const double lo = 0.5 * (static_cast<double>(s) + static_cast<double>(next_dn(s)));
        if (hi * hi < dd) {
            s = next_up(s);
        } else if (lo * lo > dd) {
            s = next_dn(s);
        } else {
            break;
        }
    }
    return s;
}

__device__ float cr_rcp(float s) {
    float r = __fdiv_rn(1.0f, s);
    if (!(s > 0.0f) || !isfinite(s) || !(r > 0.0f) || !isfinite(r)) return r;
    const double sd = s;
    for (int it = 0; it < 4; ++it) {
        const double hi = 0.5 * (static_cast<double>(r) + static_cast<double>(next_up(r)));
        const double lo = 0.5 * (static_cast<double>(r) + static_cast<double>(next_dn(r)));
        if (hi * sd < 1.0) {
            r = next_up(r);
        } else if (lo * sd > 1.0) {
            r = next_dn(r);
        } else {
            break;
        }
    }
    return r;
}

// Loads VEC consecutive entries starting at index q (VEC = 4: q is a multiple
// of 4 and the arrays are 16-byte aligned, so the 16-byte granule holding a
// valid entry is readable even past the array's end).
template <int VEC, typename T>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, int q, T (&out)[VEC]) {
    if constexpr (VEC == 4) {
        using V4 = typename std::conditional<std::is_same<T, float>::value, float4, int4>::type;
        const V4 v = *reinterpret_cast<const V4*>(p + q);
        out[0] = v.x;
        out[1] = v.y;
        out[2] = v.z;
        out[3] = v.w;
    } else {
        out[0] = p[q];
    }
}

// Per row of A (n x n): has_diag, first position (row order) of a column > i,
// the row length of A + I, and -- for gcn_norm -- the degree (sequential fp32
// sum of A + I's row values, in row order) and 1/sqrt(deg).
//
// The degree.  When every value of the row (after the diagonal's +1) is an
// integer and the sum of their magnitudes is at most 2^24, every partial sum
// of any order is an exactly representable integer, so the row's sum in any
// order equals the reference's sequential fp32 sum: the group adds them in
// parallel (in int64).  Other rows take the sequential path in row order.
// Each lane of the 16-lane group reads VEC consecutive entries per step.
template <bool NORM, int VEC>
__global__ __launch_bounds__(256) void self_loop_info_kernel(
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_ind,
    const float* __restrict__ val, int64_t n, int32_t* __restrict__ first_ins,
    int32_t* __restrict__ new_len, float* __restrict__ deg_out, float* __restrict__ dis_out) {
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (row >= n) return;
    const int b = row_ptr[row], e = row_ptr[row + 1];
    if (e - b > kLongRow) return;  // self_loop_info_long_kernel
    const int32_t i = static_cast<int32_t>(row);
    int has = 0;
    int first_gt = e - b;  // row-relative position of the first column > i
    long long isum = 0, iabs = 0;
    int integral = 1;
    const int start = VEC == 4 ? (b & ~3) : b;
    for (int q = start + g * VEC; q < e; q += kGroup * VEC) {
        int32_t c[VEC];
        float v[VEC];
        load_vec<VEC>(col_ind, q, c);
        if constexpr (NORM) load_vec<VEC>(val, q, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const int nz = q + k;
            if (nz < b || nz >= e) continue;
            has |= (c[k] == i);
            if (c[k] > i) first_gt = min(first_gt, nz - b);
            if constexpr (NORM) {
                const float x = c[k] == i ? v[k] + 1.0f : v[k];
                const bool ok = fabsf(x) <= 16777216.0f && x == rintf(x);
                integral &= ok ? 1 : 0;
                if (ok) {
                    isum += static_cast<long long>(x);
                    iabs += static_cast<long long>(fabsf(x));
                }
            }
        }
    }
#pragma unroll
    for (int d = kGroup / 2; d > 0; d >>= 1) {
        has |= __shfl_xor(has, d, kGroup);
        first_gt = min(first_gt, __shfl_xor(first_gt, d, kGroup));
        if constexpr (NORM) {
            isum += __shfl_xor(isum, d, kGroup);
            iabs += __shfl_xor(iabs, d, kGroup);
            integral &= __shfl_xor(integral, d, kGroup);
        }
    }
    if (g == 0) {
        first_ins[row] = has ? -1 : first_gt;
        new_len[row] = (e - b) + (has ? 0 : 1);
    }
    if constexpr (NORM) {
        float d = 0.0f;
        if (integral && iabs + (has ? 0 : 1) <= (1ll << 24)) {
            d = static_cast<float>(isum + (has ? 0 : 1));
        } else {
            // Sequential sum in row order of A + I: chunks of kGroup values
            // are loaded by the group and added one by one.
            for (int base = b; base < e; base += kGroup) {
                const int nz = base + g;
                float v = 0.0f;
                if (nz < e) {
                    v = val[nz];
                    if (col_ind[nz] == i) v = v + 1.0f;
                }
                const int cnt = min(kGroup, e - base);
                for (int t = 0; t < cnt; ++t) {
                    if (!has && base - b + t == first_gt) d = d + 1.0f;
                    d = d + __shfl(v, t, kGroup);
                }
            }
            if (!has && first_gt == e - b) d = d + 1.0f;
        }
        if (g == 0) {
            const float dis = d > 0.0f ? cr_rcp(cr_sqrt(d)) : 0.0f;
            deg_out[row] = d;
            dis_out[row] = dis;
        }
    }
}

// Copies entries [b, e) of row i into A + I (shifted by one past the
// inserted diagonal at `ins`), scaled when NORM.  `lanes` threads share the
// row (this one is `lane`); each keeps kCopyUnroll granules of VEC entries in
// flight, so the loads of four steps (and then their dis[c] gathers) overlap.
// A null val_out copies the structure alone (val is then not read).
constexpr int kCopyUnroll = 4;
template <bool NORM, int VEC, int LANES>
__device__ __forceinline__ void copy_span(const int32_t* __restrict__ col_ind,
                                          const float* __restrict__ val, int b, int e, int lane,
                                          int32_t i, int ins, int ob, float dis_i,
                                          const float* __restrict__ dis,
                                          int32_t* __restrict__ col_out,
                                          float* __restrict__ val_out) {
    const bool vals = val_out != nullptr;  // null: the structure alone
    const int start = VEC == 4 ? (b & ~3) : b;
    constexpr int kStep = LANES * VEC;
    for (int q0 = start + lane * VEC; q0 < e; q0 += kStep * kCopyUnroll) {
        int32_t c[kCopyUnroll][VEC];
        float v[kCopyUnroll][VEC] = {};
        float dj[kCopyUnroll][VEC];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            const int q = q0 + u * kStep;
            if (q < e) {
                load_vec<VEC>(col_ind, q, c[u]);
                if (vals) load_vec<VEC>(val, q, v[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            const int q = q0 + u * kStep;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const int nz = q + k;
                dj[u][k] = 1.0f;
                if constexpr (NORM)
                    if (q < e && nz >= b && nz < e) dj[u][k] = dis[c[u][k]];
            }
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            const int q = q0 + u * kStep;
            if (q >= e) continue;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const int nz = q + k;
                if (nz < b || nz >= e) continue;
                const int t = nz - b;
                float x = v[u][k];
                if (c[u][k] == i) x = x + 1.0f;
                if constexpr (NORM) x = (x * dis_i) * dj[u][k];
                const int o = ob + t + ((ins >= 0 && t >= ins) ? 1 : 0);
                col_out[o] = c[u][k];
                if (vals) val_out[o] = x;
            }
        }
    }
}

// 16-byte vectors: the aligned output granules of the copy, and its input
// reads, which start wherever the output granule's first input falls (dword
// aligned only).
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4_dw __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4_dw __attribute__((ext_vector_type(4), aligned(4)));

// Row i of A + I written in output order: output entry t (0 <= t < len,
// len = row length + 1 when the diagonal is inserted at `ins` >= 0) is the
// diagonal when t == ins, else input entry b + t - (ins >= 0 && t > ins).
// Lanes take 16-byte aligned granules of 4 output entries (col_out and
// val_out 16-byte aligned), kCopyUnroll per step.  A granule inside the row
// and clear of the inserted diagonal reads its 4 inputs as one vector per
// array and stores one aligned vector per array; the row's first and last
// granules (shared with the neighbouring rows) and the diagonal's go entry
// by entry.  Values: x = v (+1 on the diagonal), with NORM (x * dis_i) *
// dis[col]; the inserted diagonal is x = 1.  A null val_out copies the
// structure alone (val is then not read).
template <bool NORM, int LANES>
__device__ __forceinline__ void copy_row_granules(const int32_t* __restrict__ col_ind,
                                                  const float* __restrict__ val, int b, int e,
                                                  int lane, int32_t i, int ins, int ob,
                                                  float dis_i, const float* __restrict__ dis,
                                                  int32_t* __restrict__ col_out,
                                                  float* __restrict__ val_out) {
    const bool vals = val_out != nullptr;  // null: the structure alone
    const int len = (e - b) + (ins >= 0 ? 1 : 0);
    const int end = ob + len;
    constexpr int kStep = LANES * 4;
    for (int o0 = (ob & ~3) + lane * 4; o0 < end; o0 += kStep * kCopyUnroll) {
        i32x4 c[kCopyUnroll];
        f32x4 v[kCopyUnroll] = {};
        f32x4 dj[kCopyUnroll];
        bool fast[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            const int o = o0 + u * kStep;
            const int t = o - ob;
            fast[u] = o < end && t >= 0 && t + 4 <= len && !(ins >= t && ins < t + 4);
            if (fast[u]) {
                const int s0 = b + t - ((ins >= 0 && t > ins) ? 1 : 0);
                c[u] = *reinterpret_cast<const i32x4_dw*>(col_ind + s0);
                if (vals) v[u] = *reinterpret_cast<const f32x4_dw*>(val + s0);
            } else if (o < end) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int tk = t + k;
                    // entries outside the row (not stored) and the inserted
                    // diagonal read as (i, 0): x = 0 + 1 on the diagonal
                    int32_t ck = i;
                    float vk = 0.0f;
                    if (tk >= 0 && tk < len && tk != ins) {
                        const int src = b + tk - ((ins >= 0 && tk > ins) ? 1 : 0);
                        ck = col_ind[src];
                        if (vals) vk = val[src];
                    }
                    c[u][k] = ck;
                    v[u][k] = vk;
                }
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int u = 0; u < kCopyUnroll; ++u) {
                if (o0 + u * kStep < end) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) dj[u][k] = dis[c[u][k]];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            const int o = o0 + u * kStep;
            if (o >= end) continue;
            f32x4 x;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float xk = v[u][k];
                if (c[u][k] == i) xk = xk + 1.0f;
                if constexpr (NORM) xk = (xk * dis_i) * dj[u][k];
                x[k] = xk;
            }
            if (fast[u]) {
                *reinterpret_cast<i32x4*>(col_out + o) = c[u];
                if (vals) *reinterpret_cast<f32x4*>(val_out + o) = x;
            } else {
                const int t = o - ob;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (t + k >= 0 && t + k < len) {
                        col_out[o + k] = c[u][k];
                        if (vals) val_out[o + k] = x[k];
                    }
                }
            }
        }
    }
}

// Copies A into A + I: out position of input entry t of row i is
// row_ptr_out[i] + t (+1 past the inserted diagonal).  With NORM the values
// are scaled: ((v) * dis_i) * dis_j.  VEC = 4: aligned output granules
// (copy_row_granules; col_out and val_out 16-byte aligned); VEC = 1: one
// entry per lane and step.
template <bool NORM, int VEC>
__global__ __launch_bounds__(256) void self_loop_copy_kernel(
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_ind,
    const float* __restrict__ val, int64_t n, const int32_t* __restrict__ first_ins,
    const int32_t* __restrict__ row_ptr_out, const float* __restrict__ dis,
    int32_t* __restrict__ col_out, float* __restrict__ val_out) {
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (row >= n) return;
    const int b = row_ptr[row], e = row_ptr[row + 1];
    if (e - b > kLongRow) return;  // self_loop_copy_long_kernel
    const int32_t i = static_cast<int32_t>(row);
    const int ins = first_ins[row];
    const int ob = row_ptr_out[row];
    float dis_i = 1.0f;
    if constexpr (NORM) dis_i = dis[row];
    if constexpr (VEC == 4) {
        copy_row_granules<NORM, kGroup>(col_ind, val, b, e, g, i, ins, ob, dis_i, dis, col_out,
                                        val_out);
    } else {
        copy_span<NORM, VEC, kGroup>(col_ind, val, b, e, g, i, ins, ob, dis_i, dis, col_out,
                                     val_out);
        if (g == 0 && ins >= 0) {
            float x = 1.0f;
            if constexpr (NORM) x = (1.0f * dis_i) * dis_i;
            col_out[ob + ins] = i;
            if (val_out) val_out[ob + ins] = x;
        }
    }
}

// gcn_norm's degree and 1/sqrt(degree) for an A whose values are all 1 and
// which has no diagonal: every row of A + I sums to its length + 1, exactly
// (the integral case of self_loop_info_kernel), when that is at most 2^24;
// a longer row sets *flag (its fp32 sequential sum would saturate).
__global__ __launch_bounds__(256) void unit_dis_kernel(const int32_t* __restrict__ row_ptr,
                                                       int64_t n, float* __restrict__ dis,
                                                       int32_t* __restrict__ flag) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const int64_t d = static_cast<int64_t>(row_ptr[r + 1] - row_ptr[r]) + 1;
    if (d > (int64_t(1) << 24)) atomicOr(flag, 1);
    dis[r] = cr_rcp(cr_sqrt(static_cast<float>(d)));
}

// Rows longer than kLongRow, listed for the workgroup-per-row kernels
// (list[0..*count)); count starts at zero.
__global__ __launch_bounds__(256) void long_rows_kernel(const int32_t* __restrict__ row_ptr,
                                                        int64_t n, int32_t* __restrict__ list,
                                                        int32_t* __restrict__ count) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < n && row_ptr[r + 1] - row_ptr[r] > kLongRow)
        list[atomicAdd(count, 1)] = static_cast<int32_t>(r);
}

template <typename T>
__device__ __forceinline__ T block_reduce(T v, T* lds, int op) {  // op: 0 sum, 1 min, 2 or/and
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const T o = __shfl_xor(v, d, kWave);
        v = op == 0 ? v + o : op == 1 ? (o < v ? o : v) : (v & o);
    }
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    v = lds[0];
    for (int w = 1; w < kLongBlock / kWave; ++w)
        v = op == 0 ? v + lds[w] : op == 1 ? (lds[w] < v ? lds[w] : v) : (v & lds[w]);
    return v;
}

// self_loop_info for the listed long rows: one workgroup per row (grid-stride
// over the list).  The sequential degree (rows that fail the integral test)
// stages 1,024 values of A + I in LDS per step and adds them in row order on
// one thread.
template <bool NORM, int VEC>
__global__ __launch_bounds__(kLongBlock) void self_loop_info_long_kernel(
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_ind,
    const float* __restrict__ val, const int32_t* __restrict__ list,
    const int32_t* __restrict__ count, int32_t* __restrict__ first_ins,
    int32_t* __restrict__ new_len, float* __restrict__ deg_out, float* __restrict__ dis_out) {
    __shared__ long long red64[kLongBlock / kWave];
    __shared__ int red32[kLongBlock / kWave];
    __shared__ float stage[kLongBlock * 4];
    const int n_long = *count;
    for (int li = blockIdx.x; li < n_long; li += gridDim.x) {
        const int32_t i = list[li];
        const int b = row_ptr[i], e = row_ptr[i + 1];
        int has = 0, first_gt = e - b, integral = 1;
        long long isum = 0, iabs = 0;
        const int start = VEC == 4 ? (b & ~3) : b;
        for (int q = start + static_cast<int>(threadIdx.x) * VEC; q < e; q += kLongBlock * VEC) {
            int32_t c[VEC];
            float v[VEC];
            load_vec<VEC>(col_ind, q, c);
            if constexpr (NORM) load_vec<VEC>(val, q, v);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const int nz = q + k;
                if (nz < b || nz >= e) continue;
                has |= (c[k] == i);
                if (c[k] > i) first_gt = min(first_gt, nz - b);
                if constexpr (NORM) {
                    const float x = c[k] == i ? v[k] + 1.0f : v[k];
                    const bool ok = fabsf(x) <= 16777216.0f && x == rintf(x);
                    integral &= ok ? 1 : 0;
                    if (ok) {
                        isum += static_cast<long long>(x);
                        iabs += static_cast<long long>(fabsf(x));
                    }
                }
            }
        }
        has = block_reduce(has, red32, 0) != 0 ? 1 : 0;
        first_gt = block_reduce(first_gt, red32, 1);
        if (threadIdx.x == 0) {
            first_ins[i] = has ? -1 : first_gt;
            new_len[i] = (e - b) + (has ? 0 : 1);
        }
        if constexpr (NORM) {
            integral = block_reduce(integral, red32, 2);
            isum = block_reduce(isum, red64, 0);
            iabs = block_reduce(iabs, red64, 0);
            float d = 0.0f;
            if (integral && iabs + (has ? 0 : 1) <= (1ll << 24)) {
                d = static_cast<float>(isum + (has ? 0 : 1));
            } else {
                for (int base = b; base < e; base += kLongBlock * 4) {
                    const int cnt = min(kLongBlock * 4, e - base);
                    __syncthreads();
                    for (int t = threadIdx.x; t < cnt; t += kLongBlock) {
                        float x = val[base + t];
                        if (col_ind[base + t] == i) x = x + 1.0f;
                        stage[t] = x;
                    }
                    __syncthreads();
                    if (threadIdx.x == 0) {
                        for (int t = 0; t < cnt; ++t) {
                            if (!has && base - b + t == first_gt) d = d + 1.0f;
                            d = d + stage[t];
                        }
                    }
                }
                if (!has && first_gt == e - b) d = d + 1.0f;
            }
            if (threadIdx.x == 0) {
                deg_out[i] = d;
                dis_out[i] = d > 0.0f ? cr_rcp(cr_sqrt(d)) : 0.0f;
            }
        }
        __syncthreads();
    }
}

// self_loop_copy for the listed long rows: one workgroup per row.
template <bool NORM, int VEC>
__global__ __launch_bounds__(kLongBlock) void self_loop_copy_long_kernel(
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_ind,
    const float* __restrict__ val, const int32_t* __restrict__ list,
    const int32_t* __restrict__ count, const int32_t* __restrict__ first_ins,
    const int32_t* __restrict__ row_ptr_out, const float* __restrict__ dis,
    int32_t* __restrict__ col_out, float* __restrict__ val_out) {
    const int n_long = *count;
    for (int li = blockIdx.x; li < n_long; li += gridDim.x) {
        const int32_t i = list[li];
        const int b = row_ptr[i], e = row_ptr[i + 1];
        const int ins = first_ins[i];
        const int ob = row_ptr_out[i];
        float dis_i = 1.0f;
        if constexpr (NORM) dis_i = dis[i];
        if constexpr (VEC == 4) {
            copy_row_granules<NORM, kLongBlock>(col_ind, val, b, e, static_cast<int>(threadIdx.x),
                                                i, ins, ob, dis_i, dis, col_out, val_out);
        } else {
            copy_span<NORM, VEC, kLongBlock>(col_ind, val, b, e, static_cast<int>(threadIdx.x), i,
                                             ins, ob, dis_i, dis, col_out, val_out);
            if (threadIdx.x == 0 && ins >= 0) {
                float x = 1.0f;
                if constexpr (NORM) x = (1.0f * dis_i) * dis_i;
                col_out[ob + ins] = i;
                if (val_out) val_out[ob + ins] = x;
            }
        }
    }
}

unsigned grid_for(int64_t n, int per_block = 256, int64_t cap = 1 << 20) {
    int64_t b = ceil_div(n, per_block);
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return static_cast<unsigned>(b);
}

// Workspace layout of edge_list_to_csr.
struct CsrWs {
    int32_t* deg;
    int32_t* lists;
    int32_t* counts;
    unsigned long long* bad;
    int64_t* scan;
};

CsrWs carve_csr_ws(Carver& c, int64_t n) {
    CsrWs w{};
    w.deg = c.take<int32_t>(n + 1);
    w.lists = c.take<int32_t>(4 * n);
    w.counts = c.take<int32_t>(4);
    w.bad = c.take<unsigned long long>(1);
    w.scan = c.take<int64_t>(scan_temp_elems(n));
    return w;
}

// Sorts every row of col_ind (row_ptr given) ascending.  counts: host copy
// of the four class sizes; lists: device class lists (n entries each).
void sort_rows(int64_t n, const int32_t* row_ptr, int32_t* col, const int32_t* lists,
               const int32_t* counts, hipStream_t s) {
    if (counts[0] > 0) {
        const int64_t threads = static_cast<int64_t>(counts[0]) * kWave;
        sort_wave_kernel<<<static_cast<unsigned>(ceil_div(threads, 256)), 256, 0, s>>>(
            lists, counts[0], row_ptr, col);
        TG_LAUNCH_CHECK();
    }
    if (counts[1] > 0) {
        sort_block_kernel<256, kSortBlockMax><<<counts[1], 256, 0, s>>>(lists + n, row_ptr, col);
        TG_LAUNCH_CHECK();
    }
    if (counts[2] > 0) {
        sort_block_kernel<1024, kSortBigMax><<<counts[2], 1024, 0, s>>>(lists + 2 * n, row_ptr,
                                                                       col);
        TG_LAUNCH_CHECK();
    }
    const int n_long = counts[3];
    if (n_long == 0) return;
    // Long rows: padded lengths are needed on the host to plan the stages.
    std::vector<int32_t> rows(n_long);
    TG_HIP(hipMemcpyAsync(rows.data(), lists + 3 * n, n_long * sizeof(int32_t),
                          hipMemcpyDeviceToHost, s));
    std::vector<int32_t> rp(static_cast<size_t>(n) + 1);
    TG_HIP(hipMemcpyAsync(rp.data(), row_ptr, rp.size() * sizeof(int32_t), hipMemcpyDeviceToHost,
                          s));
    TG_HIP(hipStreamSynchronize(s));
    std::vector<int64_t> seg_off(n_long + 1, 0), tile_off, tile_len;
    int64_t pmax = 0;
    for (int i = 0; i < n_long; ++i) {
        const int len = rp[rows[i] + 1] - rp[rows[i]];
        const int64_t pad = next_pow2(len);  // >= 32768, a multiple of the tile
        seg_off[i + 1] = seg_off[i] + pad;
        pmax = std::max(pmax, pad);
        for (int64_t t = 0; t < pad / kSortTile; ++t) {
            tile_off.push_back(seg_off[i]);
            tile_len.push_back(pad);
        }
    }
    const int64_t total = seg_off[n_long];
    const int64_t n_tiles = total / kSortTile;
    require(pmax <= (int64_t(1) << 30) && n_long < 65536,
            "GraphLoader::edge_list_to_csr: row too long for the device sort");
    Carver probe(nullptr, 0);
    probe.take<int32_t>(total);
    probe.take<int64_t>(n_long + 1);
    probe.take<int64_t>(n_tiles);
    probe.take<int64_t>(n_tiles);
    probe.take<int32_t>(n_long);
    DeviceBuffer buf(probe.bytes());
    Carver c(buf.get(), buf.size());
    int32_t* tmp = c.take<int32_t>(total);
    int64_t* d_seg = c.take<int64_t>(n_long + 1);
    int64_t* d_toff = c.take<int64_t>(n_tiles);
    int64_t* d_tlen = c.take<int64_t>(n_tiles);
    int32_t* d_rows = c.take<int32_t>(n_long);
    TG_HIP(hipMemcpyAsync(d_seg, seg_off.data(), seg_off.size() * sizeof(int64_t),
                          hipMemcpyHostToDevice, s));
    TG_HIP(hipMemcpyAsync(d_toff, tile_off.data(), n_tiles * sizeof(int64_t),
                          hipMemcpyHostToDevice, s));
    TG_HIP(hipMemcpyAsync(d_tlen, tile_len.data(), n_tiles * sizeof(int64_t),
                          hipMemcpyHostToDevice, s));
    TG_HIP(hipMemcpyAsync(d_rows, rows.data(), n_long * sizeof(int32_t), hipMemcpyHostToDevice,
                          s));
    dim3 g2(static_cast<unsigned>(std::min<int64_t>(ceil_div(pmax, 256), 1024)),
            static_cast<unsigned>(n_long));
    long_gather_kernel<<<g2, 256, 0, s>>>(d_rows, d_seg, n_long, row_ptr, col, tmp);
    TG_LAUNCH_CHECK();
    // stages k <= tile inside each tile
    long_tile_kernel<<<static_cast<unsigned>(n_tiles), 1024, 0, s>>>(tmp, d_toff, d_tlen, 0, 2,
                                                                     kSortTile, 1);
    TG_LAUNCH_CHECK();
    for (int64_t k = 2 * kSortTile; k <= pmax; k <<= 1) {
        for (int64_t j = k >> 1; j >= kSortTile; j >>= 1) {
            long_step_kernel<<<grid_for(total, 256, 65536), 256, 0, s>>>(tmp, d_toff, d_tlen,
                                                                         total, k, j);
            TG_LAUNCH_CHECK();
        }
        // remaining distances j < tile of stage k, tile-local
        long_tile_kernel<<<static_cast<unsigned>(n_tiles), 1024, 0, s>>>(
            tmp, d_toff, d_tlen, k, static_cast<int>(k), static_cast<int>(k), kSortTile / 2);
        TG_LAUNCH_CHECK();
    }
    long_scatter_kernel<<<g2, 256, 0, s>>>(d_rows, d_seg, n_long, row_ptr, col, tmp);
    TG_LAUNCH_CHECK();
    TG_HIP(hipStreamSynchronize(s));  // `buf` is released on return
}

void require_square(int64_t n, const char* fn) {
    require(n >= 0, std::string(fn) + ": negative size");
    require(n < (int64_t(1) << 31), std::string(fn) + ": n must be < 2^31 (int32 CSR)");
}

// Shared by add_self_loops and gcn_norm.
// values = false: row_ptr_out and col_out only (val_out is ignored; with
// norm, deg_out / dis_out are still computed).
void self_loops_impl(bool norm, int64_t n, int64_t nnz, const int32_t* row_ptr,
                     const int32_t* col_ind, const float* val, int32_t* row_ptr_out,
                     int32_t* col_out, float* val_out, float* deg_out, float* dis_out,
                     void* workspace, size_t ws_bytes, hipStream_t s, bool values) {
    const char* fn = norm ? "gcn_norm" : "add_self_loops";
    require_square(n, fn);
    require(nnz >= 0 && nnz + n < (int64_t(1) << 31),
            std::string(fn) + ": nnz + n must be < 2^31 (int32 CSR)");
    if (n == 0) {
        write_i32_kernel<<<1, 1, 0, s>>>(row_ptr_out, 0);
        TG_LAUNCH_CHECK();
        return;
    }
    if (!values) val_out = nullptr;
    require(row_ptr && row_ptr_out && col_out && (val_out || !values),
            std::string(fn) + ": null pointer");
    require(nnz == 0 || (col_ind && val), std::string(fn) + ": null pointer");
    Carver probe(nullptr, 0);
    probe.take<int32_t>(n);
    probe.take<int32_t>(n + 1);
    probe.take<float>(n);
    probe.take<float>(n);
    probe.take<int64_t>(scan_temp_elems(n));
    probe.take<int32_t>(n + 1);  // long-row list + its count
    DeviceBuffer own;
    if (workspace == nullptr) {
        own.resize(probe.bytes());
        workspace = own.get();
        ws_bytes = own.size();
    }
    Carver c(workspace, ws_bytes);
    int32_t* first_ins = c.take<int32_t>(n);
    int32_t* new_len = c.take<int32_t>(n + 1);
    float* deg = c.take<float>(n);
    float* dis = c.take<float>(n);
    int64_t* scan = c.take<int64_t>(scan_temp_elems(n));
    int32_t* long_list = c.take<int32_t>(n + 1);
    int32_t* long_count = long_list + n;
    if (deg_out) deg = deg_out;
    if (dis_out) dis = dis_out;
    const unsigned blocks = static_cast<unsigned>(ceil_div(n * kGroup, 256));
    fill_i32(long_count, 1, 0, s);
    long_rows_kernel<<<grid_for(n), 256, 0, s>>>(row_ptr, n, long_list, long_count);
    TG_LAUNCH_CHECK();
    const unsigned long_grid = 8192;  // grid-stride over the (device-side) long-row list
    // 128-bit reads when both arrays are 16-byte aligned
    const bool v4 = (reinterpret_cast<uintptr_t>(col_ind) | reinterpret_cast<uintptr_t>(val)) % 16 == 0;
    if (norm && v4)
        self_loop_info_kernel<true, 4><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n, first_ins,
                                                              new_len, deg, dis);
    else if (norm)
        self_loop_info_kernel<true, 1><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n, first_ins,
                                                              new_len, deg, dis);
    else if (v4)
        self_loop_info_kernel<false, 4><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n,
                                                               first_ins, new_len, nullptr,
                                                               nullptr);
    else
        self_loop_info_kernel<false, 1><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n,
                                                               first_ins, new_len, nullptr,
                                                               nullptr);
    TG_LAUNCH_CHECK();
    if (norm && v4)
        self_loop_info_long_kernel<true, 4><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, new_len, deg, dis);
    else if (norm)
        self_loop_info_long_kernel<true, 1><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, new_len, deg, dis);
    else if (v4)
        self_loop_info_long_kernel<false, 4><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, new_len, nullptr, nullptr);
    else
        self_loop_info_long_kernel<false, 1><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, new_len, nullptr, nullptr);
    TG_LAUNCH_CHECK();
    exclusive_scan_i32(new_len, row_ptr_out, n, scan, s);
    // the copy writes 128-bit granules when both outputs are 16-byte aligned
    const bool o4 = (reinterpret_cast<uintptr_t>(col_out) | reinterpret_cast<uintptr_t>(val_out)) % 16 == 0;
    // the structure alone needs no scaling: copied as add_self_loops' structure
    const bool scale = norm && values;
    if (scale && o4)
        self_loop_copy_kernel<true, 4><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n, first_ins,
                                                              row_ptr_out, dis, col_out, val_out);
    else if (scale)
        self_loop_copy_kernel<true, 1><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n, first_ins,
                                                              row_ptr_out, dis, col_out, val_out);
    else if (o4)
        self_loop_copy_kernel<false, 4><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n,
                                                               first_ins, row_ptr_out, nullptr,
                                                               col_out, val_out);
    else
        self_loop_copy_kernel<false, 1><<<blocks, 256, 0, s>>>(row_ptr, col_ind, val, n,
                                                               first_ins, row_ptr_out, nullptr,
                                                               col_out, val_out);
    TG_LAUNCH_CHECK();
    if (scale && o4)
        self_loop_copy_long_kernel<true, 4><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, row_ptr_out, dis, col_out,
            val_out);
    else if (scale)
        self_loop_copy_long_kernel<true, 1><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, row_ptr_out, dis, col_out,
            val_out);
    else if (o4)
        self_loop_copy_long_kernel<false, 4><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, row_ptr_out, nullptr,
            col_out, val_out);
    else
        self_loop_copy_long_kernel<false, 1><<<long_grid, kLongBlock, 0, s>>>(
            row_ptr, col_ind, val, long_list, long_count, first_ins, row_ptr_out, nullptr,
            col_out, val_out);
    TG_LAUNCH_CHECK();
    if (own.get()) TG_HIP(hipStreamSynchronize(s));  // own workspace is freed on return
}

size_t self_loops_ws(int64_t n) {
    Carver c(nullptr, 0);
    c.take<int32_t>(n);
    c.take<int32_t>(n + 1);
    c.take<float>(n);
    c.take<float>(n);
    c.take<int64_t>(scan_temp_elems(n));
    c.take<int32_t>(n + 1);
    return c.bytes();
}

}  // namespace

// Host entry used by the C-ABI and the Model.
void edge_list_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src, const int32_t* dst,
                      int32_t* row_ptr, int32_t* col_ind, float* val, void* workspace,
                      size_t ws_bytes, hipStream_t s, bool check_dst, const char* who) {
    const std::string W = who ? who : "GraphLoader::edge_list_to_csr";
    require(n_nodes >= 0 && n_edges >= 0, W + ": negative size");
    if (n_nodes == 0) {
        require(n_edges == 0, W + ": num_nodes is 0 but edges is non-empty");
        write_i32_kernel<<<1, 1, 0, s>>>(row_ptr, 0);
        TG_LAUNCH_CHECK();
        return;
    }
    require(n_nodes < (int64_t(1) << 31) && n_edges < (int64_t(1) << 31),
            W + ": sizes must be < 2^31 (int32 CSR)");
    require(row_ptr != nullptr, W + ": row_ptr is null");
    require(n_edges == 0 || (src && dst && col_ind && val),
            W + ": null pointer");
    Carver probe(nullptr, 0);
    carve_csr_ws(probe, n_nodes);
    DeviceBuffer own;
    if (workspace == nullptr) {
        own.resize(probe.bytes());
        workspace = own.get();
        ws_bytes = own.size();
    }
    Carver c(workspace, ws_bytes);
    CsrWs w = carve_csr_ws(c, n_nodes);
    fill_i32(w.deg, n_nodes, 0, s);
    fill_i32(w.counts, 4, 0, s);
    fill_i32(reinterpret_cast<int32_t*>(w.bad), 2, -1, s);  // UINT64_MAX
    if (n_edges > 0) {
        edge_count_kernel<<<grid_for(n_edges, 256, 16384), 256, 0, s>>>(
            src, dst, n_edges, static_cast<int32_t>(n_nodes), check_dst ? 1 : 0, w.deg, w.bad);
        TG_LAUNCH_CHECK();
    }
    classify_rows_kernel<<<grid_for(n_nodes), 256, 0, s>>>(w.deg, n_nodes, w.lists, w.counts);
    TG_LAUNCH_CHECK();
    unsigned long long bad = 0;
    int32_t counts[4];
    TG_HIP(hipMemcpyAsync(&bad, w.bad, sizeof(bad), hipMemcpyDeviceToHost, s));
    TG_HIP(hipMemcpyAsync(counts, w.counts, sizeof(counts), hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    if (bad != ~0ull) {
        const int64_t e = static_cast<int64_t>(bad / 2);
        const bool is_dst = (bad & 1) != 0;
        int32_t v = 0;
        TG_HIP(hipMemcpy(&v, (is_dst ? dst : src) + e, sizeof(v), hipMemcpyDeviceToHost));
        throw std::invalid_argument(W + ": edge[" + std::to_string(e) +
                                    "]." + (is_dst ? "dst" : "src") + " = " +
                                    std::to_string(v) + " out of range [0, " +
                                    std::to_string(n_nodes) + ")");
    }
    exclusive_scan_i32(w.deg, row_ptr, n_nodes, w.scan, s);
    if (n_edges > 0) {
        fill_i32(w.deg, n_nodes, 0, s);  // reused as the per-row cursor
        edge_scatter_kernel<<<grid_for(n_edges, 256, 16384), 256, 0, s>>>(
            src, dst, n_edges, row_ptr, w.deg, col_ind, val);
        TG_LAUNCH_CHECK();
        sort_rows(n_nodes, row_ptr, col_ind, w.lists, counts, s);
    }
    if (own.get()) TG_HIP(hipStreamSynchronize(s));
}

size_t edge_list_to_csr_ws(int64_t n_nodes) {
    Carver c(nullptr, 0);
    carve_csr_ws(c, n_nodes);
    return c.bytes();
}

void csr_validate(int64_t n_rows, int64_t n_cols, int64_t nnz, const int32_t* row_ptr,
                  const int32_t* col_ind, hipStream_t s) {
    require(n_rows >= 0 && n_cols >= 0 && nnz >= 0, "Tensor::sparse_csr: negative size");
    require(row_ptr != nullptr, "Tensor::sparse_csr: row_ptr is null");
    require(nnz == 0 || col_ind != nullptr, "Tensor::sparse_csr: col_ind is null");
    int32_t last = 0;
    TG_HIP(hipMemcpyAsync(&last, row_ptr + n_rows, sizeof(last), hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    // tensor.cpp:61-67 converts row_ptr.back() to size_t before comparing
    if (static_cast<std::size_t>(last) != static_cast<std::size_t>(nnz))
        throw std::invalid_argument("Tensor::sparse_csr: row_ptr.back() (" +
                                    std::to_string(static_cast<std::size_t>(last)) +
                                    ") must equal values.size() (" + std::to_string(nnz) + ")");
    DeviceBuffer b(2 * sizeof(unsigned long long));
    auto* bad = b.as<unsigned long long>();
    fill_i32(reinterpret_cast<int32_t*>(bad), 4, -1, s);
    csr_check_kernel<<<grid_for(std::max(nnz, n_rows + 1), 256, 16384), 256, 0, s>>>(
        row_ptr, n_rows, col_ind, nnz, n_cols, bad);
    TG_LAUNCH_CHECK();
    unsigned long long h[2];
    TG_HIP(hipMemcpyAsync(h, bad, sizeof(h), hipMemcpyDeviceToHost, s));
    TG_HIP(hipStreamSynchronize(s));
    if (h[0] != ~0ull) {
        int32_t v = 0;
        TG_HIP(hipMemcpy(&v, col_ind + h[0], sizeof(v), hipMemcpyDeviceToHost));
        throw std::invalid_argument("Tensor::sparse_csr: col_ind[" + std::to_string(h[0]) +
                                    "] = " + std::to_string(v) +
                                    " is out of bounds for cols=" + std::to_string(n_cols));
    }
    if (h[1] != ~0ull) {
        int32_t v[2];
        TG_HIP(hipMemcpy(v, row_ptr + h[1] - 1, sizeof(v), hipMemcpyDeviceToHost));
        throw std::invalid_argument(
            "Tensor::sparse_csr: row_ptr must be non-decreasing; row_ptr[" +
            std::to_string(h[1]) + "] = " + std::to_string(v[1]) + " < row_ptr[" +
            std::to_string(h[1] - 1) + "] = " + std::to_string(v[0]));
    }
}

void add_self_loops(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
                    const float* val, int32_t* row_ptr_out, int32_t* col_out, float* val_out,
                    void* ws, size_t ws_bytes, hipStream_t s, bool values) {
    self_loops_impl(false, n, nnz, row_ptr, col_ind, val, row_ptr_out, col_out, val_out, nullptr,
                    nullptr, ws, ws_bytes, s, values);
}

void gcn_norm(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
              const float* val, int32_t* row_ptr_out, int32_t* col_out, float* val_out,
              float* deg_out, float* dis_out, void* ws, size_t ws_bytes, hipStream_t s,
              bool values) {
    self_loops_impl(true, n, nnz, row_ptr, col_ind, val, row_ptr_out, col_out, val_out, deg_out,
                    dis_out, ws, ws_bytes, s, values);
}

size_t self_loops_workspace(int64_t n) { return self_loops_ws(n); }

void unit_self_loop_dis(int64_t n, const int32_t* row_ptr, float* dis, int32_t* flag,
                        hipStream_t s) {
    if (n == 0) return;
    unit_dis_kernel<<<static_cast<unsigned>(ceil_div(n, 256)), 256, 0, s>>>(row_ptr, n, dis, flag);
    TG_LAUNCH_CHECK();
}

}  // namespace tg

extern "C" {

size_t tg_edge_list_to_csr_workspace_size(int64_t n_nodes, int64_t n_edges) {
    (void)n_edges;
    return n_nodes > 0 ? tg::edge_list_to_csr_ws(n_nodes) : 0;
}

int tg_edge_list_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src, const int32_t* dst,
                        int32_t* row_ptr, int32_t* col_ind, float* val, void* workspace,
                        size_t workspace_bytes, tg_stream_t stream) {
    return tg::guard([&] {
        tg::edge_list_to_csr(n_nodes, n_edges, src, dst, row_ptr, col_ind, val, workspace,
                             workspace_bytes, static_cast<hipStream_t>(stream), true, nullptr);
    });
}

int tg_coo_to_csr(int64_t n_nodes, int64_t n_edges, const int32_t* src, const int32_t* dst,
                  int32_t* row_ptr, int32_t* col_ind, float* val, const char* context,
                  tg_stream_t stream) {
    return tg::guard([&] {
        const auto s = static_cast<hipStream_t>(stream);
        const std::string who = context ? context : "coo_to_csr";
        tg::edge_list_to_csr(n_nodes, n_edges, src, dst, row_ptr, col_ind, val, nullptr, 0, s,
                             /*check_dst=*/false, who.c_str());
        tg::csr_validate(n_nodes, n_nodes, n_edges, row_ptr, col_ind, s);
        TG_HIP(hipStreamSynchronize(s));
    });
}

int tg_csr_validate(int64_t n_rows, int64_t n_cols, int64_t nnz, const int32_t* row_ptr,
                    const int32_t* col_ind, tg_stream_t stream) {
    return tg::guard([&] {
        tg::csr_validate(n_rows, n_cols, nnz, row_ptr, col_ind, static_cast<hipStream_t>(stream));
    });
}

size_t tg_self_loops_workspace_size(int64_t n) { return n > 0 ? tg::self_loops_workspace(n) : 0; }

int tg_add_self_loops(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
                      const float* val, int32_t* row_ptr_out, int32_t* col_ind_out,
                      float* val_out, void* workspace, size_t workspace_bytes,
                      tg_stream_t stream) {
    return tg::guard([&] {
        tg::add_self_loops(n, nnz, row_ptr, col_ind, val, row_ptr_out, col_ind_out, val_out,
                           workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                           true);
    });
}

int tg_gcn_norm(int64_t n, int64_t nnz, const int32_t* row_ptr, const int32_t* col_ind,
                const float* val, int32_t* row_ptr_out, int32_t* col_ind_out, float* val_out,
                float* deg_out, float* dis_out, void* workspace, size_t workspace_bytes,
                tg_stream_t stream) {
    return tg::guard([&] {
        tg::gcn_norm(n, nnz, row_ptr, col_ind, val, row_ptr_out, col_ind_out, val_out, deg_out,
                     dis_out, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                     true);
    });
}

}  // extern "C"
