// Causal grouped-query attention of the training step as batched matmuls plus per-query-row chains
// (nn.hpp:535-615 forward, grad.hpp:206-301 backward), for every window and head of a step at once.
//
// Layout: scores are kept transposed, S^T[j][t] (key j, query t) per (window, head), so the columns a query owns are
// contiguous across queries: the softmax chains (first maximum, exponentials, their serial total; the backward's
// D = sum_j p_j dp_j) run one lane per query over keys ascending, with coalesced loads, and the matmuls find their
// wave-uniform operand rows contiguous.
//
//   forward   S^T = K Q^T * scale   (double, head_dim ascending, exact float products: fma)
//             E^T = exp(S^T - max_t), total_t serial, inv_t = 1 / total_t       (one lane per query)
//             out[t] = f32((sum_j E^T[j][t] v[j]) * inv_t)                         (keys ascending, multiply then add)
//   backward  P^T = E^T * inv_t;  dP^T = V dOut^T (double, exact products)
//             D_t = sum_j p dp (serial), dS^T = p (dp - D) scale                     (one lane per query)
//             dq[t] = f32(sum_j dS[t][j] k[j])                                       (keys ascending)
//             dk[j] = f32(sum over (t ascending, head of the group ascending) dS q), dv[j] likewise with p and dOut
// Each reduction runs exactly over the keys (or queries) the reference visits, in its order: rows of a tile that
// see fewer keys are predicated off the extra steps, never fed zeros.
#include "attn_gemm.h"
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

constexpr int kTI = 16;    // wave-uniform rows per wave
constexpr int kWaves = 4;  // waves per workgroup, stacked along rows

struct Operand {
    const void* ptr;
    int64_t w_stride, seg_stride, head_stride;  // base = ptr + w*w_stride + seg[w]*seg_stride + (hz/head_div)*head_stride
    int64_t head_div;
    int64_t ld, ld_inner, group;  // row(l) = (l / group) * ld + (l % group) * ld_inner
};

template <typename T>
__device__ __forceinline__ const T* base_of(const Operand& o, int64_t w, int64_t seg_w, int64_t hz) {
    return static_cast<const T*>(o.ptr) + w * o.w_stride + seg_w * o.seg_stride + (hz / o.head_div) * o.head_stride;
}

struct AttnGemmParams {
    Operand A, B, C;
    const double* rowscale;  // per (z, row) multiplier before rounding (out = acc * inv); may be null
    int64_t rowscale_zstride;
    const int64_t* seg;
    int64_t heads;    // z = w * heads + hz
    int rows_kind;    // I = n_w (positions) if 0, head_dim if 1
    int cols_kind;    // J = n_w if 0, head_dim if 1
    int64_t head_dim;
    int64_t group;    // G for the key-row limits
    int mask;         // kMaskNone, kMaskQueryRows, kMaskKeyRows, kMaskTileCausal
    int64_t window;
    int64_t L;        // reduction length when unmasked (head_dim)
    double out_scale; // double outputs: value = acc * out_scale
};

// The keys query t sees (causal, q_offset 0, optional window): [lo, hi).
__device__ __forceinline__ void query_span(int64_t t, int64_t window, int64_t* lo, int64_t* hi) {
    *hi = t + 1;
    *lo = window != 0 && t + 1 > window ? t + 1 - window : 0;
}

// The (t, head-in-group) rows that see key j, as l = t * G + hh: [lo, hi).
__device__ __forceinline__ void key_span(int64_t j, int64_t n, int64_t window, int64_t G, int64_t* lo, int64_t* hi) {
    *lo = j * G;
    const int64_t t_hi = window != 0 && j + window - 1 < n - 1 ? j + window - 1 : n - 1;
    *hi = (t_hi + 1) * G;
}

template <int CJ>
__device__ __forceinline__ void load_cols(const float* row, int64_t j0, int64_t J, float out[CJ]) {
#pragma unroll
    for (int c = 0; c < CJ; ++c) out[c] = row[j0 + c < J ? j0 + c : J - 1];
}

template <int CJ, bool kFma, bool kPredicated>
__device__ __forceinline__ void run_steps(const double* __restrict__ A, int64_t lda, const float* __restrict__ B,
                                          const Operand& bo, int64_t i0, int64_t j0, int64_t J, int64_t l_begin,
                                          int64_t l_end, const int64_t lo[kTI], const int64_t hi[kTI],
                                          double acc[kTI][CJ]) {
    int64_t t = l_begin / bo.group, hh = l_begin % bo.group;
    for (int64_t l = l_begin; l < l_end; ++l) {
        const float* brow = B + t * bo.ld + hh * bo.ld_inner;
        float bv[CJ];
        load_cols<CJ>(brow, j0, J, bv);
        const double* arow = A + l * lda + i0;
#pragma unroll
        for (int q = 0; q < kTI; ++q) {
            const double a = arow[q];
            if (kPredicated && !(l >= lo[q] && l < hi[q])) continue;
#pragma unroll
            for (int c = 0; c < CJ; ++c) {
                if (kFma)
                    acc[q][c] = __builtin_fma(a, static_cast<double>(bv[c]), acc[q][c]);
                else
                    acc[q][c] = acc[q][c] + a * static_cast<double>(bv[c]);
            }
        }
        if (++hh == bo.group) {
            hh = 0;
            ++t;
        }
    }
}

template <int CJ, bool kFma, bool kOutDouble>
__global__ __launch_bounds__(256) void attn_gemm_kernel(AttnGemmParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t z = blockIdx.z;
    const int64_t w = z / p.heads, hz = z % p.heads;
    const int64_t seg_w = p.seg[w], n = p.seg[w + 1] - seg_w;
    const int64_t I = p.rows_kind == 0 ? n : p.head_dim;
    const int64_t J = p.cols_kind == 0 ? n : p.head_dim;
    const int64_t i0 = (static_cast<int64_t>(blockIdx.y) * kWaves + wave) * kTI;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * 64 * CJ + lane * CJ;
    const int64_t jw0 = static_cast<int64_t>(blockIdx.x) * 64 * CJ;  // first column of the wave
    if (i0 >= I || jw0 >= J) return;  // wave-uniform
    if (p.mask == kMaskTileCausal) {
        // S^T / dP^T tiles: rows are keys j, columns queries t; a tile no query of which sees any of its keys is skipped
        const int64_t t_last = jw0 + 64 * CJ - 1;
        if (i0 > t_last) return;
        if (p.window != 0 && i0 + kTI - 1 + p.window - 1 < jw0) return;
    }
    int64_t lo[kTI], hi[kTI];
    int64_t l_begin = 0, l_end = p.L, common_lo = 0, common_hi = p.L;
    if (p.mask == kMaskQueryRows || p.mask == kMaskKeyRows) {
        l_begin = INT64_MAX;
        l_end = 0;
        common_lo = 0;
        common_hi = INT64_MAX;
#pragma unroll
        for (int q = 0; q < kTI; ++q) {
            const int64_t r = i0 + q < I ? i0 + q : I - 1;
            if (p.mask == kMaskQueryRows)
                query_span(r, p.window, &lo[q], &hi[q]);
            else
                key_span(r, n, p.window, p.group, &lo[q], &hi[q]);
            l_begin = lo[q] < l_begin ? lo[q] : l_begin;
            l_end = hi[q] > l_end ? hi[q] : l_end;
            common_lo = lo[q] > common_lo ? lo[q] : common_lo;
            common_hi = hi[q] < common_hi ? hi[q] : common_hi;
        }
        if (common_lo > common_hi) common_lo = common_hi = l_begin;  // no step shared by all rows
    } else {
#pragma unroll
        for (int q = 0; q < kTI; ++q) {
            lo[q] = 0;
            hi[q] = p.L;
        }
    }
    const double* A = base_of<double>(p.A, w, seg_w, hz);
    const float* B = base_of<float>(p.B, w, seg_w, hz);
    double acc[kTI][CJ];
#pragma unroll
    for (int q = 0; q < kTI; ++q)
#pragma unroll
        for (int c = 0; c < CJ; ++c) acc[q][c] = 0.0;
    if (common_lo > l_begin) run_steps<CJ, kFma, true>(A, p.A.ld, B, p.B, i0, j0, J, l_begin, common_lo, lo, hi, acc);
    run_steps<CJ, kFma, false>(A, p.A.ld, B, p.B, i0, j0, J, common_lo, common_hi, lo, hi, acc);
    if (l_end > common_hi) run_steps<CJ, kFma, true>(A, p.A.ld, B, p.B, i0, j0, J, common_hi, l_end, lo, hi, acc);
#pragma unroll
    for (int q = 0; q < kTI; ++q) {
        const int64_t i = i0 + q;
        if (i >= I) break;
#pragma unroll
        for (int c = 0; c < CJ; ++c) {
            const int64_t j = j0 + c;
            if (j >= J) continue;
            if (kOutDouble) {
                double* C = const_cast<double*>(base_of<double>(p.C, w, seg_w, hz));
                C[i * p.C.ld + j] = acc[q][c] * p.out_scale;
            } else {
                float* C = const_cast<float*>(base_of<float>(p.C, w, seg_w, hz));
                double v = acc[q][c];
                if (p.rowscale) v = v * p.rowscale[z * p.rowscale_zstride + i];
                C[i * p.C.ld + j] = static_cast<float>(v);
            }
        }
    }
}

// One lane per query t of a (window, head): the forward softmax chains over its visible keys (nn.hpp:541-561):
// first maximum, then e = exp(s - max) written back over S^T and their serial total; inv_t = 1 / total.
__global__ __launch_bounds__(64) void softmax_rows_kernel(double* __restrict__ st, int64_t ld, int64_t zstride,
                                                          const int64_t* __restrict__ seg, int64_t heads,
                                                          int64_t window, double* __restrict__ inv,
                                                          int64_t inv_zstride) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    double* s = st + z * zstride;
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    double mx = s[lo * ld + t];
    for (int64_t j = lo + 1; j < hi; ++j) {
        const double v = s[j * ld + t];
        if (v > mx) mx = v;
    }
    double total = 0.0;
    for (int64_t j = lo; j < hi; ++j) {
        const double e = dexp(s[j * ld + t] - mx);
        s[j * ld + t] = e;
        total += e;
    }
    inv[z * inv_zstride + t] = 1.0 / total;
}

// Backward chains per query (grad.hpp:262-278): p = e * inv (over E^T, in place), D = sum p dp (serial), and
// ds = (p (dp - D)) scale over dP^T in place.
__global__ __launch_bounds__(64) void dsoftmax_rows_kernel(double* __restrict__ et, double* __restrict__ dpt,
                                                           int64_t ld, int64_t zstride,
                                                           const int64_t* __restrict__ seg, int64_t heads,
                                                           int64_t window, const double* __restrict__ inv,
                                                           int64_t inv_zstride, double scale) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    double* e = et + z * zstride;
    double* d = dpt + z * zstride;
    const double iv = inv[z * inv_zstride + t];
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    double weighted = 0.0;
    for (int64_t j = lo; j < hi; ++j) {
        const double pj = e[j * ld + t] * iv;
        e[j * ld + t] = pj;
        weighted += pj * d[j * ld + t];
    }
    for (int64_t j = lo; j < hi; ++j) d[j * ld + t] = e[j * ld + t] * (d[j * ld + t] - weighted) * scale;
}

// dst[w][g][(t * G + hh)][j] = src[w][g * G + hh][j][t] (doubles): the key-row operand layout of dk / dv.
__global__ __launch_bounds__(256) void regroup_kernel(const double* __restrict__ src, int64_t ld, int64_t zstride,
                                                      double* __restrict__ dst, int64_t dst_ld, int64_t dst_zstride,
                                                      const int64_t* __restrict__ seg, int64_t heads, int64_t group) {
    __shared__ double tile[64][65];
    const int64_t z = blockIdx.z;  // (w, h)
    const int64_t w = z / heads, h = z % heads;
    const int64_t g = h / group, hh = h % group;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t j0 = static_cast<int64_t>(blockIdx.y) * 64, t0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (j0 >= n || t0 >= n) return;
    const double* s = src + z * zstride;
    double* d = dst + (w * (heads / group) + g) * dst_zstride;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t j = j0 + k, t = t0 + tx;
        tile[k][tx] = (j < n && t < n) ? s[j * ld + t] : 0.0;
    }
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, j = j0 + tx;
        if (t < n && j < n) d[(t * group + hh) * dst_ld + j] = tile[tx][k];
    }
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

int launch_attn_gemm(const AttnGemmCall& c, hipStream_t stream) {
    AttnGemmParams p;
    auto op = [](const AttnOperand& o) {
        return Operand{o.ptr, o.w_stride, o.seg_stride, o.head_stride, o.head_div > 0 ? o.head_div : 1, o.ld,
                       o.ld_inner, o.group > 0 ? o.group : 1};
    };
    p.A = op(c.A);
    p.B = op(c.B);
    p.C = op(c.C);
    p.rowscale = c.rowscale;
    p.rowscale_zstride = c.rowscale_zstride;
    p.seg = c.seg;
    p.heads = c.heads;
    p.rows_kind = c.rows_kind;
    p.cols_kind = c.cols_kind;
    p.head_dim = c.head_dim;
    p.group = c.group > 0 ? c.group : 1;
    p.mask = c.mask;
    p.window = c.window;
    p.L = c.L;
    p.out_scale = c.out_scale;
    const int64_t I = c.rows_kind == 0 ? c.max_len : c.head_dim;
    const int64_t J = c.cols_kind == 0 ? c.max_len : c.head_dim;
    const int cj = c.cols_per_lane;
    DLLM_REQUIRE(cj == 2 || cj == 4, "columns per lane must be 2 or 4");
    dim3 grid(static_cast<unsigned>(ceil_div(J, 64 * cj)), static_cast<unsigned>(ceil_div(I, kTI * kWaves)),
              static_cast<unsigned>(c.windows * c.heads));
    if (I == 0 || J == 0 || grid.z == 0) return kOk;
#define DLLM_ATTN_LAUNCH(CJ, FMA, OUTD)                                                                 \
    hipLaunchKernelGGL((attn_gemm_kernel<CJ, FMA, OUTD>), grid, dim3(256), 0, stream, p)
    if (cj == 4 && c.exact_products && c.out_double) DLLM_ATTN_LAUNCH(4, true, true);
    else if (cj == 4 && c.exact_products) DLLM_ATTN_LAUNCH(4, true, false);
    else if (cj == 4 && c.out_double) DLLM_ATTN_LAUNCH(4, false, true);
    else if (cj == 4) DLLM_ATTN_LAUNCH(4, false, false);
    else if (c.exact_products && c.out_double) DLLM_ATTN_LAUNCH(2, true, true);
    else if (c.exact_products) DLLM_ATTN_LAUNCH(2, true, false);
    else if (c.out_double) DLLM_ATTN_LAUNCH(2, false, true);
    else DLLM_ATTN_LAUNCH(2, false, false);
#undef DLLM_ATTN_LAUNCH
    return check_launch("attention matmul");
}

int launch_softmax_rows(double* st, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                        int64_t max_len, int64_t window, double* inv, int64_t inv_zstride, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(softmax_rows_kernel, grid, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                       inv_zstride);
    return check_launch("attention softmax");
}

int launch_dsoftmax_rows(double* et, double* dpt, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows,
                         int64_t heads, int64_t max_len, int64_t window, const double* inv, int64_t inv_zstride,
                         double scale, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(dsoftmax_rows_kernel, grid, dim3(64), 0, stream, et, dpt, ld, zstride, seg, heads, window, inv,
                       inv_zstride, scale);
    return check_launch("attention softmax backward");
}

int launch_regroup(const double* src, int64_t ld, int64_t zstride, double* dst, int64_t dst_ld, int64_t dst_zstride,
                   const int64_t* seg, int64_t windows, int64_t heads, int64_t group, int64_t max_len,
                   hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(max_len, 64)),
              static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(regroup_kernel, grid, dim3(256), 0, stream, src, ld, zstride, dst, dst_ld, dst_zstride, seg,
                       heads, group);
    return check_launch("attention regroup");
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
