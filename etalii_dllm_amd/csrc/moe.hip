// Mixture-of-experts routing and its float32 glue (cpp/include/dllm/nn.hpp:864-896, grad.hpp:507-541,
// src/etalii_dllm/training/backprop.py:308-377, 501-527).
//
//   moe_route           per row: softmax (math.hpp:387-398: max, e = exp(l - max) in double, total ascending,
//                       p = f32(e * (1 / total))), then the k largest p in a total order (ties to the lower expert),
//                       optionally divided by their double total in rank order
//   moe_route_backward  per row: dp = dprob (or 0); for each chosen e: dp[e] += dw / S - C / S^2 (normalize) or dw,
//                       S = sum of chosen p, C = sum of dw p (rank order); D = sum over e of p dp (ascending);
//                       dlogits = f32(p (dp - D))
//   combine             out[r] = (((0 + t_0) + t_1) + ...) + addend[r], one term per choice of row r in ascending
//                       expert order: t = f32(y w) for the expert outputs, t = dx for the input gradients
//   router statistics   per window: mean[e] = f32(sum over layers, then rows, of p[e] / rows) (column_mean,
//                       interp.hpp:146-155), loss = E * dot(f32(count / rows), mean), grad[e] = f32(s E count / rows^2)
//
// The per-row chains are serial, as in the reference, one lane per row. Each probability is recomputed where it is
// needed from the row's max and total (exp is deterministic), so no per-row scratch is kept.
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

struct RowSoftmax {
    double max = 0.0, inv = 0.0;
};

// argmax keeps the first of equal values (math.hpp:376-385); the max value itself is all that is used
__device__ RowSoftmax row_softmax(const float* __restrict__ l, int64_t E) {
    float m = l[0];
    for (int64_t e = 1; e < E; ++e)
        if (l[e] > m) m = l[e];
    RowSoftmax s;
    s.max = static_cast<double>(m);
    double total = 0.0;
    for (int64_t e = 0; e < E; ++e) total += dexp(static_cast<double>(l[e]) - s.max);
    s.inv = 1.0 / total;
    return s;
}

__device__ __forceinline__ float row_prob(const float* __restrict__ l, const RowSoftmax& s, int64_t e) {
    return static_cast<float>(dexp(static_cast<double>(l[e]) - s.max) * s.inv);
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int64_t rows, int64_t E,
                                                        int64_t K, int normalize, int64_t* __restrict__ indices,
                                                        float* __restrict__ weights, float* __restrict__ probs) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= rows) return;
    const float* l = logits + r * E;
    const RowSoftmax s = row_softmax(l, E);
    if (probs)
        for (int64_t e = 0; e < E; ++e) probs[r * E + e] = row_prob(l, s, e);
    double total = 0.0;
    for (int64_t j = 0; j < K; ++j) {
        int64_t best = E;
        float pb = 0.0f;
        for (int64_t e = 0; e < E; ++e) {
            bool taken = false;
            for (int64_t i = 0; i < j; ++i) taken = taken || indices[r * K + i] == e;
            if (taken) continue;
            const float p = row_prob(l, s, e);
            if (best == E || p > pb) {
                best = e;
                pb = p;
            }
        }
        indices[r * K + j] = best;
        weights[r * K + j] = pb;
        total += static_cast<double>(pb);
    }
    if (normalize)
        for (int64_t j = 0; j < K; ++j)
            weights[r * K + j] = static_cast<float>(static_cast<double>(weights[r * K + j]) / total);
}

__global__ __launch_bounds__(256) void moe_route_backward_kernel(const float* __restrict__ logits,
                                                                 const int64_t* __restrict__ indices,
                                                                 const float* __restrict__ dweights,
                                                                 const float* __restrict__ dprob, int64_t rows,
                                                                 int64_t E, int64_t K, int normalize,
                                                                 float* __restrict__ dlogits) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= rows) return;
    const float* l = logits + r * E;
    const int64_t* idx = indices + r * K;
    const float* dw = dweights + r * K;
    const RowSoftmax s = row_softmax(l, E);
    double total = 0.0, weighted = 0.0;
    for (int64_t j = 0; j < K; ++j) {
        const double p = static_cast<double>(row_prob(l, s, idx[j]));
        total += p;
        weighted += static_cast<double>(dw[j]) * p;
    }
    // dp[e] = dprob[e] (+ the term of the rank choosing e; an expert is chosen at most once per row)
    auto dp_of = [&](int64_t e) {
        double dp = dprob ? static_cast<double>(dprob[r * E + e]) : 0.0;
        for (int64_t j = 0; j < K; ++j)
            if (idx[j] == e) {
                const double d = static_cast<double>(dw[j]);
                dp += normalize ? d / total - weighted / (total * total) : d;
            }
        return dp;
    };
    double dot = 0.0;
    for (int64_t e = 0; e < E; ++e) dot += static_cast<double>(row_prob(l, s, e)) * dp_of(e);
    for (int64_t e = 0; e < E; ++e)
        dlogits[r * E + e] = static_cast<float>(static_cast<double>(row_prob(l, s, e)) * (dp_of(e) - dot));
}

// out[r][d] = (0 + sum over the row's choices in expert order of term) + addend[r][d]; term = y[p][d] * w (weights
// given) or y[p][d]. order[r * K + i] is the grouped position p of the row's i-th choice by expert, slot[p] its
// index into the routing weights.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y, const int64_t* __restrict__ order,
                                                          const int64_t* __restrict__ slot,
                                                          const float* __restrict__ weights,
                                                          const float* __restrict__ addend, float* __restrict__ out,
                                                          int64_t rows, int64_t K, int64_t H) {
    const int64_t n = rows * H;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / H, d = i - r * H;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const int64_t p = order[r * K + k];
            const float v = y[p * H + d];
            acc = acc + (weights ? v * weights[slot[p]] : v);
        }
        out[i] = acc + addend[i];
    }
}

// Per grouped position p (row r = row_of[p], routing slot q = slot[p]):
//   dweights[q] = f32(sum over d ascending of dout[r][d] y[p][d])   (dllm::dot, one lane per position)
//   dy[p][d]    = dout[r][d] * weights[q]
// A workgroup takes 64 positions; its four waves stage 64-column tiles of the products in LDS (writing dy on the
// way), then wave 0 runs the 64 chains.
__global__ __launch_bounds__(256) void moe_dweights_kernel(const float* __restrict__ dout, const float* __restrict__ y,
                                                           const int64_t* __restrict__ row_of,
                                                           const int64_t* __restrict__ slot,
                                                           const float* __restrict__ weights, int64_t positions,
                                                           int64_t H, float* __restrict__ dweights,
                                                           float* __restrict__ dy) {
    __shared__ double prod[64][65];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t np = positions - p0 < 64 ? positions - p0 : 64;
    double chain = 0.0;
    for (int64_t c0 = 0; c0 < H; c0 += 64) {
        const int n = static_cast<int>(H - c0 < 64 ? H - c0 : 64);
        if (lane < n) {
            for (int k = 0; k < 16; ++k) {
                const int q = wave * 16 + k;
                if (q < np) {
                    const int64_t p = p0 + q;
                    const float g = dout[row_of[p] * H + c0 + lane];
                    prod[q][lane] = static_cast<double>(g) * static_cast<double>(y[p * H + c0 + lane]);
                    dy[p * H + c0 + lane] = g * weights[slot[p]];
                }
            }
        }
        __syncthreads();
        if (wave == 0 && lane < np)
            for (int c = 0; c < n; ++c) chain += prod[lane][c];
        __syncthreads();
    }
    if (wave == 0 && lane < np) dweights[slot[p0 + lane]] = static_cast<float>(chain);
}

// One workgroup per window w: rows = (seg[w + 1] - seg[w]) * layers; probs of layer l at probs + l * layer_stride.
// Each expert's mean is one serial chain over (layer, row) ascending; the rows reach the chains through LDS in
// chunks of kStatRows (x E floats) that the whole workgroup loads ahead, so the chains wait on LDS, not on HBM.
constexpr int kStatFloats = 8192;  // floats per LDS chunk

__global__ __launch_bounds__(256) void router_stats_kernel(const float* __restrict__ probs, int64_t layer_stride,
                                                           int64_t layers, const int64_t* __restrict__ seg,
                                                           const int64_t* __restrict__ counts, int64_t E,
                                                           double router_scale, double* __restrict__ loss,
                                                           float* __restrict__ grad_row) {
    __shared__ float chunk[2][kStatFloats];
    __shared__ float frac_mean[2 * 8192];  // [E] fractions, [E] means
    const int64_t w = blockIdx.x;
    const int64_t r0 = seg[w], n = seg[w + 1] - r0;
    const int64_t rows = n * layers;
    const int64_t* cnt = counts + w * E;
    const int tid = static_cast<int>(threadIdx.x);
    const int64_t per = E <= kStatFloats ? kStatFloats / E : 1;  // rows per chunk
    // an expert's chain lives in thread e % 256 (experts e, e + 256, ...); 32 chains per thread at most
    double total[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) total[k] = 0.0;
    const int64_t chunks = (rows + per - 1) / per;
    // element f of chunk c: row q = c per + f / E (layer q / n, row q % n of the window), expert f % E
    const uint32_t E32 = static_cast<uint32_t>(E), n32 = static_cast<uint32_t>(n > 0 ? n : 1);
    auto load = [&](int64_t c, float (&reg)[kStatFloats / 256]) {
#pragma unroll
        for (int k = 0; k < kStatFloats / 256; ++k) {
            const uint32_t f = static_cast<uint32_t>(k * 256 + tid);
            const uint32_t fr = f / E32;
            const int64_t q = c * per + fr;
            const uint32_t l = static_cast<uint32_t>(q) / n32;
            reg[k] = (fr < per && q < rows)
                         ? probs[l * layer_stride + (r0 + (static_cast<uint32_t>(q) - l * n32)) * E + (f - fr * E32)]
                         : 0.0f;
        }
    };
    float reg[kStatFloats / 256];
    if (chunks > 0) {
        load(0, reg);
#pragma unroll
        for (int k = 0; k < kStatFloats / 256; ++k) chunk[0][k * 256 + tid] = reg[k];
    }
    __syncthreads();
    for (int64_t c = 0; c < chunks; ++c) {
        if (c + 1 < chunks) load(c + 1, reg);  // in flight while the chains run
        const float* cur = chunk[c & 1];
        const int64_t in_chunk = rows - c * per < per ? rows - c * per : per;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const int64_t e = tid + 256 * k;
            if (e >= E) break;
            double t = total[k];
            for (int64_t q = 0; q < in_chunk; ++q) t += static_cast<double>(cur[q * E + e]);
            total[k] = t;
        }
        if (c + 1 < chunks) {
#pragma unroll
            for (int k = 0; k < kStatFloats / 256; ++k) chunk[(c + 1) & 1][k * 256 + tid] = reg[k];
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int64_t e = tid + 256 * k;
        if (e >= E) break;
        frac_mean[E + e] = rows > 0 ? static_cast<float>(total[k] / static_cast<double>(rows)) : 0.0f;
    }
    for (int64_t e = tid; e < E; e += 256) {
        frac_mean[e] = static_cast<float>(static_cast<double>(cnt[e]) / static_cast<double>(rows));
        if (grad_row)
            grad_row[w * E + e] = static_cast<float>(router_scale * static_cast<double>(E) *
                                                     static_cast<double>(cnt[e]) / static_cast<double>(rows * rows));
    }
    __syncthreads();
    if (tid == 0) {
        double acc = 0.0;
        for (int64_t e = 0; e < E; ++e)
            acc += static_cast<double>(frac_mean[e]) * static_cast<double>(frac_mean[E + e]);
        loss[w] = static_cast<double>(E) * static_cast<double>(static_cast<float>(acc));
    }
}

// dprob[r] = grad_row[window of r] for every row of every window.
__global__ __launch_bounds__(256) void broadcast_rows_kernel(const float* __restrict__ grad_row,
                                                             const int64_t* __restrict__ seg, int nseg, int64_t E,
                                                             float* __restrict__ out) {
    const int64_t r = blockIdx.x;
    int w = 0;
    while (w + 1 < nseg && seg[w + 1] <= r) ++w;
    for (int64_t e = threadIdx.x; e < E; e += 256) out[r * E + e] = grad_row[w * E + e];
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ logits, float* __restrict__ out,
                                                           int64_t rows, int64_t n) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= rows) return;
    const RowSoftmax s = row_softmax(logits + r * n, n);
    for (int64_t e = 0; e < n; ++e) out[r * n + e] = row_prob(logits + r * n, s, e);
}

__global__ __launch_bounds__(256) void column_mean_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                          int64_t rows, int64_t cols) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    double total = 0.0;
    for (int64_t r = 0; r < rows; ++r) total += static_cast<double>(x[r * cols + c]);
    out[c] = rows > 0 ? static_cast<float>(total / static_cast<double>(rows)) : 0.0f;
}

__global__ void dot_kernel(const float* __restrict__ a, const float* __restrict__ b, int64_t n,
                           float* __restrict__ result) {
    if (threadIdx.x != 0) return;
    double acc = 0.0;
    for (int64_t i = 0; i < n; ++i) acc += static_cast<double>(a[i]) * static_cast<double>(b[i]);
    *result = static_cast<float>(acc);
}

unsigned row_grid(int64_t rows) { return static_cast<unsigned>(ceil_div(static_cast<size_t>(rows), 256)); }

}  // namespace

int launch_moe_route(const float* logits, int64_t rows, int64_t experts, int64_t k, int normalize, int64_t* indices,
                     float* weights, float* probs, hipStream_t stream) {
    DLLM_REQUIRE(k >= 1 && k <= experts, "experts per token must be between 1 and the number of experts");
    if (rows == 0) return kOk;
    hipLaunchKernelGGL(moe_route_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, logits, rows, experts, k,
                       normalize, indices, weights, probs);
    return check_launch("moe_route");
}

int launch_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights, const float* dprob,
                              int64_t rows, int64_t experts, int64_t k, int normalize, float* dlogits,
                              hipStream_t stream) {
    DLLM_REQUIRE(k >= 1 && k <= experts, "indices must be [rows, k] with k between 1 and the number of experts");
    if (rows == 0) return kOk;
    hipLaunchKernelGGL(moe_route_backward_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, logits, indices,
                       dweights, dprob, rows, experts, k, normalize, dlogits);
    return check_launch("moe_route_backward");
}

int launch_moe_combine(const float* y, const int64_t* order, const int64_t* slot, const float* weights,
                       const float* addend, float* out, int64_t rows, int64_t k, int64_t dim, hipStream_t stream) {
    const int64_t n = rows * dim;
    if (n == 0) return kOk;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 256), 16384));
    hipLaunchKernelGGL(moe_combine_kernel, dim3(blocks), dim3(256), 0, stream, y, order, slot, weights, addend, out,
                       rows, k, dim);
    return check_launch("moe_combine");
}

int launch_moe_dweights(const float* dout, const float* y, const int64_t* row_of, const int64_t* slot,
                        const float* weights, int64_t positions, int64_t dim, float* dweights, float* dy,
                        hipStream_t stream) {
    if (positions == 0) return kOk;
    hipLaunchKernelGGL(moe_dweights_kernel, dim3(static_cast<unsigned>(ceil_div(positions, 64))), dim3(256), 0, stream,
                       dout, y, row_of, slot, weights, positions, dim, dweights, dy);
    return check_launch("moe_dweights");
}

int launch_router_stats(const float* probs, int64_t layer_stride, int64_t layers, const int64_t* seg, int nseg,
                        const int64_t* counts, int64_t experts, double router_scale, double* loss, float* grad_row,
                        hipStream_t stream) {
    DLLM_REQUIRE(experts <= 8192, "too many experts for the router statistics");
    if (nseg == 0) return kOk;
    hipLaunchKernelGGL(router_stats_kernel, dim3(static_cast<unsigned>(nseg)), dim3(256), 0, stream, probs,
                       layer_stride, layers, seg, counts, experts, router_scale, loss, grad_row);
    return check_launch("router_stats");
}

int launch_softmax_rows(const float* logits, float* out, int64_t rows, int64_t n, hipStream_t stream) {
    DLLM_REQUIRE(n >= 1, "softmax needs at least one value");
    if (rows == 0) return kOk;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, logits, out, rows, n);
    return check_launch("softmax");
}

int launch_column_mean(const float* x, float* out, int64_t rows, int64_t cols, hipStream_t stream) {
    if (cols == 0) return kOk;
    hipLaunchKernelGGL(column_mean_kernel, dim3(row_grid(cols)), dim3(256), 0, stream, x, out, rows, cols);
    return check_launch("column_mean");
}

int launch_dot(const float* a, const float* b, int64_t n, float* result, hipStream_t stream) {
    hipLaunchKernelGGL(dot_kernel, dim3(1), dim3(64), 0, stream, a, b, n, result);
    return check_launch("dot");
}

int launch_broadcast_window_rows(const float* grad_row, const int64_t* seg, int nseg, int64_t rows, int64_t experts,
                                 float* out, hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(rows <= 2147483647, "too many rows");
    hipLaunchKernelGGL(broadcast_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, grad_row, seg,
                       nseg, experts, out);
    return check_launch("broadcast_window_rows");
}

}  // namespace dllm_hip
