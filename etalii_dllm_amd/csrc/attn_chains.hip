// The per-query chains of the training step's causal grouped-query attention (nn.hpp:535-615 forward, grad.hpp:206-301
// backward), for every window and head of a step at once; the matmuls around them are in attn_lds.hip.
//
// Layout: scores are kept transposed, S^T[j][t] (key j, query t) per (window, head), so the columns a query owns are
// contiguous across queries: the chains run one lane per query over keys ascending, with coalesced loads.
//
//   forward   E^T = exp(S^T - max_t), total_t serial, inv_t = 1 / total_t       (one kernel; max_t from the score
//             tiles' maxima when the scores kernel provides them, else a first walk; small launches split it into
//             maximum, exps and totals)
//   backward  D_t = sum over keys ascending of (e inv_t) dp (serial); p = e inv_t, dS = p (dp - D_t) scale
//             elementwise, dS written over dP^T and p, dS in the key-row layout dk / dv read (two kernels: a fused
//             one, a wave per 64 queries, measured slower, its LDS tiles limiting it to one wave per SIMD; so was
//             writing p and dS in place only, with dk / dv gathering key rows from the query-major storage: its
//             tiles took 182 against 156 ms per step at T = 2048 for 16 ms less here)
// Each chain visits exactly the keys the reference visits, in its order.
#include "attn_step.h"
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

// The keys query t of a window of n sees: causal with q_offset 0 and an optional sliding window, or every key when
// window is kAllKeys: [lo, hi).
__device__ __forceinline__ void query_span(int64_t t, int64_t n, int64_t window, int64_t* lo, int64_t* hi) {
    if (window < 0) {
        *lo = 0;
        *hi = n;
        return;
    }
    *hi = t + 1;
    *lo = window != 0 && t + 1 > window ? t + 1 - window : 0;
}

// The forward softmax of every query (nn.hpp:541-561), one lane per query over its visible keys ascending, in one
// kernel with two walks over its column of S^T (measured against separate max, exp and total passes: 54 against
// 66 ms per step at T = 2048, alike at T = 1024):
//   1. mx_t = the first maximum (strictly greater replaces)
//   2. e = exp(s - mx_t) written over S^T, and total_t = the serial sum of the e in the same order; inv_t = 1 / total_t
// The lanes' loads are issued kChainUnroll keys ahead of their serial use; 64 lanes read 64 consecutive queries of a
// key row (coalesced).
constexpr int kChainUnroll = 8;

__global__ __launch_bounds__(64) void softmax_fused_kernel(double* __restrict__ st, int64_t ld, int64_t zstride,
                                                           const int64_t* __restrict__ seg, int64_t heads,
                                                           int64_t window, double* __restrict__ inv,
                                                           int64_t inv_zstride) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    double* s = st + z * zstride + t;
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    double mx = s[lo * ld];
    int64_t j = lo + 1;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = s[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k)
            if (v[k] > mx) mx = v[k];
    }
    for (; j < hi; ++j) {
        const double v = s[j * ld];
        if (v > mx) mx = v;
    }
    double total = 0.0;
    j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = s[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) {
            const double e = dexp(v[k] - mx);
            s[(j + k) * ld] = e;
            total += e;
        }
    }
    for (; j < hi; ++j) {
        const double e = dexp(s[j * ld] - mx);
        s[j * ld] = e;
        total += e;
    }
    inv[z * inv_zstride + t] = 1.0 / total;
}

// The forward softmax with the maximum from the score tiles' maxima (attn_mfma_kernel): the value of the reference's
// first maximum is the first score when that is NaN, else the largest non-NaN score (a strictly greater one replaces
// it), which the tile maxima give in any order; e = exp(s - mx) is the same for mx = +0 and -0. Then one walk: e over
// S^T and total_t = the serial sum of the e in key order; inv_t = 1 / total_t.
__global__ __launch_bounds__(64) void softmax_tiles_kernel(double* __restrict__ st, int64_t ld, int64_t zstride,
                                                           const int64_t* __restrict__ seg, int64_t heads,
                                                           int64_t window, double* __restrict__ inv,
                                                           int64_t inv_zstride, const double* __restrict__ tile_max,
                                                           int64_t tm_zstride, int64_t tm_ld) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    double* s = st + z * zstride + t;
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    const double first = s[lo * ld];
    double mx = first;
    if (first == first) {
        const double* tm = tile_max + z * tm_zstride + t;
        mx = -__builtin_huge_val();
        for (int64_t k = lo / 64; k <= (hi - 1) / 64; ++k) {
            const double m = tm[k * tm_ld];
            if (m > mx) mx = m;
        }
    }
    double total = 0.0;
    int64_t j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = s[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) {
            const double e = dexp(v[k] - mx);
            s[(j + k) * ld] = e;
            total += e;
        }
    }
    for (; j < hi; ++j) {
        const double e = dexp(s[j * ld] - mx);
        s[j * ld] = e;
        total += e;
    }
    inv[z * inv_zstride + t] = 1.0 / total;
}

// The backward chains per query (grad.hpp:262-278) in two passes:
//   dsoftmax_dot_kernel    D_t = sum over visible keys ascending of (e inv_t) dp (one lane per query)
//   dsoftmax_apply_kernel  p = e inv_t over E^T and ds = (p (dp - D_t)) scale over dP^T (each element independent)
__global__ __launch_bounds__(64) void dsoftmax_dot_kernel(const double* __restrict__ et, const double* __restrict__ dpt,
                                                          int64_t ld, int64_t zstride,
                                                          const int64_t* __restrict__ seg, int64_t heads,
                                                          int64_t window, const double* __restrict__ inv,
                                                          int64_t inv_zstride, double* __restrict__ dvec) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    const double* e = et + z * zstride + t;
    const double* d = dpt + z * zstride + t;
    const double iv = inv[z * inv_zstride + t];
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    double weighted = 0.0;
    int64_t j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double term[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) term[k] = (e[(j + k) * ld] * iv) * d[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) weighted += term[k];
    }
    for (; j < hi; ++j) weighted += (e[j * ld] * iv) * d[j * ld];
    dvec[z * inv_zstride + t] = weighted;
}

// The elementwise part of the softmax backward with the key-row layout of dk / dv written directly: per visible
// (key j, query t) of head h = g G + hh, p = e inv_t and ds = (p (dp - D_t)) scale; ds is written over dP^T[j][t]
// (dq's operand) and p, ds to pg / dsg[w][g][(t G + hh)][j]. A 64 x 64 tile goes through LDS so both the reads
// (along t) and the regrouped writes (along j) are coalesced.
template <bool kSlope>
__global__ __launch_bounds__(256) void dsoftmax_apply_regroup_kernel(
    const double* __restrict__ et, double* __restrict__ dpt, int64_t ld, int64_t zstride,
    const int64_t* __restrict__ seg, int64_t heads, int64_t group, int64_t window, const double* __restrict__ inv,
    int64_t inv_zstride, const double* __restrict__ dvec, double scale, double* __restrict__ pg,
    double* __restrict__ dsg, int64_t dst_ld, int64_t dst_zstride, const double* __restrict__ slope) {
    constexpr int kJ = 32;  // keys per tile (64 queries)
    __shared__ double tp[kJ][65];
    __shared__ double td[kJ][65];
    const int64_t z = blockIdx.z;
    const int64_t w = z / heads, h = z % heads;
    const int64_t g = h / group, hh = h % group;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64, j0 = static_cast<int64_t>(blockIdx.y) * kJ;
    if (t0 >= n || j0 >= n || (window >= 0 && j0 > t0 + 63)) return;
    int64_t lo0, hi0;
    query_span(t0, n, window, &lo0, &hi0);
    if (j0 + kJ - 1 < lo0) return;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    {
        const int64_t t = t0 + tx;
        int64_t lo = 0, hi = 0;
        if (t < n) query_span(t, n, window, &lo, &hi);
        const double iv = t < n ? inv[z * inv_zstride + t] : 0.0;
        const double D = t < n ? dvec[z * inv_zstride + t] : 0.0;
        const double* e = et + z * zstride + t;
        double* d = dpt + z * zstride + t;
        const double* sl = kSlope ? slope + z * zstride + t : nullptr;
        double ev[kJ / 4], dv[kJ / 4], sv[kJ / 4];
#pragma unroll
        for (int k = 0; k < kJ / 4; ++k) {  // every load issued before the first use
            const int64_t j = j0 + ty + 4 * k;
            const bool vis = j >= lo && j < hi;
            ev[k] = vis ? e[j * ld] : 0.0;
            dv[k] = vis ? d[j * ld] : 0.0;
            if (kSlope) sv[k] = vis ? sl[j * ld] : 1.0;
        }
#pragma unroll
        for (int k = 0; k < kJ / 4; ++k) {
            const int64_t j = j0 + ty + 4 * k;
            if (j >= lo && j < hi) {
                const double p = ev[k] * iv;
                // ((p (dp - D)) slope) scale, the slope of a soft-capped score (1 without a cap: the product is exact)
                const double ds = kSlope ? p * (dv[k] - D) * sv[k] * scale : p * (dv[k] - D) * scale;
                d[j * ld] = ds;
                tp[ty + 4 * k][tx] = p;
                td[ty + 4 * k][tx] = ds;
            }
        }
    }
    __syncthreads();
    // writes: 32 keys of a query row per 32 lanes, two rows per wave
    const int64_t row0 = (w * (heads / group) + g) * dst_zstride;
    const int jx = threadIdx.x & 31, tr = threadIdx.x >> 5;  // tr: 0..7
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int64_t t = t0 + tr + 8 * k, j = j0 + jx;
        if (t >= n) break;
        int64_t lo, hi;
        query_span(t, n, window, &lo, &hi);
        if (j >= lo && j < hi) {
            const int64_t at = row0 + (t * group + hh) * dst_ld + j;
            pg[at] = tp[jx][tr + 8 * k];
            dsg[at] = td[jx][tr + 8 * k];
        }
    }
}

// Small launches (few windows x heads x 64-query blocks leave most of the GPU idle with one lane per query): the
// forward softmax splits so that its exps spread over the GPU. The maximum first (one lane per query, into the inv
// slot), then e = exp(s - mx) over S^T by one thread per key run, then one lane per query adds the e in key order and
// writes inv = 1 / total over the maximum. The same values and the same serial sums. (Split the same way, the
// backward's D chain measured no faster at T = 256: its terms are one multiply each.)
constexpr int64_t kSplitChainsBelow = 512;  // windows x heads x 64-query blocks (more: one walk, measured faster)
constexpr int kTermKeys = 32;                // keys per workgroup of the exp kernel (8 per wave)

__global__ __launch_bounds__(64) void softmax_max_kernel(const double* __restrict__ st, int64_t ld, int64_t zstride,
                                                         const int64_t* __restrict__ seg, int64_t heads,
                                                         int64_t window, double* __restrict__ mx_out,
                                                         int64_t inv_zstride, const double* __restrict__ tile_max,
                                                         int64_t tm_zstride, int64_t tm_ld) {
    const int64_t z = blockIdx.y;
    const int64_t n = seg[z / heads + 1] - seg[z / heads];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    const double first = st[z * zstride + lo * ld + t];
    double mx = first;
    if (first == first) {
        const double* tm = tile_max + z * tm_zstride + t;
        mx = -__builtin_huge_val();
        for (int64_t k = lo / 64; k <= (hi - 1) / 64; ++k) {
            const double m = tm[k * tm_ld];
            if (m > mx) mx = m;
        }
    }
    mx_out[z * inv_zstride + t] = mx;
}

__global__ __launch_bounds__(256) void softmax_exp_kernel(double* __restrict__ st, int64_t ld, int64_t zstride,
                                                          const int64_t* __restrict__ seg, int64_t heads,
                                                          int64_t window, const double* __restrict__ mx_in,
                                                          int64_t inv_zstride) {
    const int64_t z = blockIdx.z;
    const int64_t n = seg[z / heads + 1] - seg[z / heads];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + (threadIdx.x & 63);
    const int64_t j0 = static_cast<int64_t>(blockIdx.y) * kTermKeys + (threadIdx.x >> 6) * (kTermKeys / 4);
    if (t >= n) return;
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    if (j0 >= hi || j0 + kTermKeys / 4 <= lo) return;
    const double mx = mx_in[z * inv_zstride + t];
    double* s = st + z * zstride + t;
#pragma unroll
    for (int k = 0; k < kTermKeys / 4; ++k) {
        const int64_t j = j0 + k;
        if (j >= lo && j < hi) s[j * ld] = dexp(s[j * ld] - mx);
    }
}

__global__ __launch_bounds__(64) void softmax_total_kernel(const double* __restrict__ et, int64_t ld, int64_t zstride,
                                                           const int64_t* __restrict__ seg, int64_t heads,
                                                           int64_t window, double* __restrict__ inv,
                                                           int64_t inv_zstride) {
    const int64_t z = blockIdx.y;
    const int64_t n = seg[z / heads + 1] - seg[z / heads];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    int64_t lo, hi;
    query_span(t, n, window, &lo, &hi);
    const double* e = et + z * zstride + t;
    double total = 0.0;
    int64_t j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = e[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) total += v[k];
    }
    for (; j < hi; ++j) total += e[j * ld];
    inv[z * inv_zstride + t] = 1.0 / total;
}

// Per (window, head): dst[i][t] = src[(seg[w] + t) * row_stride + head * head_dim + i], as double or float.
template <typename T>
__global__ __launch_bounds__(256) void heads_transpose_kernel(const float* __restrict__ src, int64_t row_stride,
                                                              int64_t head_dim, T* __restrict__ dst, int64_t ld,
                                                              int64_t zstride, const int64_t* __restrict__ seg,
                                                              int64_t heads) {
    __shared__ float tile[64][65];
    const int64_t z = blockIdx.z;
    const int64_t w = z / heads, h = z % heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64, i0 = static_cast<int64_t>(blockIdx.y) * 64;
    if (t0 >= n || i0 >= head_dim) return;
    const float* s = src + seg[w] * row_stride + h * head_dim;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, i = i0 + tx;
        tile[k][tx] = (t < n && i < head_dim) ? s[t * row_stride + i] : 0.0f;
    }
    __syncthreads();
    T* d = dst + z * zstride;
    for (int k = ty; k < 64; k += 4) {
        const int64_t i = i0 + k, t = t0 + tx;
        if (i < head_dim && t < n) d[i * ld + t] = static_cast<T>(tile[tx][k]);
    }
}

}  // namespace

int launch_softmax_rows(double* st, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                        int64_t max_len, int64_t window, double* inv, int64_t inv_zstride, hipStream_t stream,
                        const double* tile_max, int64_t tile_max_zstride, int64_t tile_max_ld) {
    if (max_len == 0 || windows * heads == 0) return kOk;
    const dim3 lanes(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    if (tile_max && windows * heads * ceil_div(max_len, 64) < kSplitChainsBelow) {
        const dim3 terms(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(max_len, kTermKeys)),
                         static_cast<unsigned>(windows * heads));
        hipLaunchKernelGGL(softmax_max_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                           inv_zstride, tile_max, tile_max_zstride, tile_max_ld);
        hipLaunchKernelGGL(softmax_exp_kernel, terms, dim3(256), 0, stream, st, ld, zstride, seg, heads, window, inv,
                           inv_zstride);
        hipLaunchKernelGGL(softmax_total_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                           inv_zstride);
    } else if (tile_max)
        hipLaunchKernelGGL(softmax_tiles_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                           inv_zstride, tile_max, tile_max_zstride, tile_max_ld);
    else
        hipLaunchKernelGGL(softmax_fused_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                           inv_zstride);
    return check_launch("attention softmax");
}

__global__ __launch_bounds__(256) void softcap_scores_kernel(double* __restrict__ st, double* __restrict__ slope,
                                                             int64_t count, double cap) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const double t = dtanh(st[i] / cap);
        st[i] = cap * t;
        slope[i] = 1.0 - t * t;
    }
}

int launch_softcap_scores(double* st, double* slope, int64_t count, double cap, hipStream_t stream) {
    if (count == 0) return kOk;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(count, 256), 16384));
    hipLaunchKernelGGL(softcap_scores_kernel, dim3(blocks), dim3(256), 0, stream, st, slope, count, cap);
    return check_launch("softcap scores");
}

int launch_dsoftmax_regroup(const double* et, double* dpt, int64_t ld, int64_t zstride, const int64_t* seg,
                            int64_t windows, int64_t heads, int64_t group, int64_t max_len, int64_t window,
                            const double* inv, int64_t inv_zstride, double scale, double* dvec, double* pg,
                            double* dsg, int64_t dst_ld, int64_t dst_zstride, hipStream_t stream,
                            const double* slope) {
    if (max_len == 0 || windows * heads == 0) return kOk;
    const dim3 lanes(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(dsoftmax_dot_kernel, lanes, dim3(64), 0, stream, et, dpt, ld, zstride, seg, heads, window, inv,
                       inv_zstride, dvec);
    const dim3 tiles(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(max_len, 32)),
                     static_cast<unsigned>(windows * heads));
    if (slope)
        hipLaunchKernelGGL(dsoftmax_apply_regroup_kernel<true>, tiles, dim3(256), 0, stream, et, dpt, ld, zstride, seg,
                           heads, group, window, inv, inv_zstride, dvec, scale, pg, dsg, dst_ld, dst_zstride, slope);
    else
        hipLaunchKernelGGL(dsoftmax_apply_regroup_kernel<false>, tiles, dim3(256), 0, stream, et, dpt, ld, zstride,
                           seg, heads, group, window, inv, inv_zstride, dvec, scale, pg, dsg, dst_ld, dst_zstride,
                           nullptr);
    return check_launch("attention softmax backward");
}

int launch_heads_transpose(const float* src, int64_t row_stride, int64_t head_dim, void* dst, bool to_double,
                           int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                           int64_t max_len, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(head_dim, 64)),
              static_cast<unsigned>(windows * heads));
    if (to_double)
        hipLaunchKernelGGL(heads_transpose_kernel<double>, grid, dim3(256), 0, stream, src, row_stride, head_dim,
                           static_cast<double*>(dst), ld, zstride, seg, heads);
    else
        hipLaunchKernelGGL(heads_transpose_kernel<float>, grid, dim3(256), 0, stream, src, row_stride, head_dim,
                           static_cast<float*>(dst), ld, zstride, seg, heads);
    return check_launch("heads transpose");
}

}  // namespace dllm_hip
