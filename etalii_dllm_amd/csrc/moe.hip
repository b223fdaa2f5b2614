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
#include <algorithm>

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

// Rows of at most 256 experts run one wave per row (expert e = lane + 64 m on lane `lane`), the row's probabilities
// in registers. moe_route_wave_kernel: rank j takes the first untaken expert when its p is NaN (nothing is greater
// than NaN), else the largest untaken non-NaN p, the lower expert on ties: the reference's scan in which only a
// strictly greater p replaces the best.
constexpr int kRouteLanesPer = 4;

__device__ __forceinline__ double readlane_f64(double v, int k) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), k));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), k));
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// The row's probabilities in a wave, pv[m] for expert lane + 64 m (row_softmax and row_prob restated: the maximum's
// value is the first logit when that is NaN, else the largest non-NaN one; the total is the serial sum over e
// ascending, read lane by lane).
__device__ __forceinline__ void wave_row_probs(const float* __restrict__ l, int64_t E, int lane,
                                               float (&pv)[kRouteLanesPer]) {
    float lv[kRouteLanesPer];
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) {
        const int64_t e = lane + 64 * m;
        lv[m] = e < E ? l[e] : 0.0f;
    }
    const float first = __shfl(lv[0], 0, 64);
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m)
        if (lane + 64 * m < E && lv[m] > mx) mx = lv[m];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off, 64);
        mx = o > mx ? o : mx;
    }
    if (first != first) mx = first;
    const double dmax = static_cast<double>(mx);
    double ev[kRouteLanesPer];
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m)
        ev[m] = lane + 64 * m < E ? dexp(static_cast<double>(lv[m]) - dmax) : 0.0;
    double total = 0.0;
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) {
        if (64 * m >= E) break;
        const int n = E - 64 * m < 64 ? static_cast<int>(E - 64 * m) : 64;
        for (int k = 0; k < n; ++k) total += readlane_f64(ev[m], k);
    }
    const double inv = 1.0 / total;
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) pv[m] = static_cast<float>(ev[m] * inv);
}

// the probability of expert e (uniform across the wave)
__device__ __forceinline__ float wave_prob(const float (&pv)[kRouteLanesPer], int64_t e) {
    const int l = static_cast<int>(e & 63), mm = static_cast<int>(e >> 6);
    float p = 0.0f;
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m)
        if (m == mm) p = __shfl(pv[m], l, 64);
    return p;
}

__global__ __launch_bounds__(256) void moe_route_wave_kernel(const float* __restrict__ logits, int64_t rows,
                                                             int64_t E, int64_t K, int normalize,
                                                             int64_t* __restrict__ indices,
                                                             float* __restrict__ weights, float* __restrict__ probs) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float pv[kRouteLanesPer];
    wave_row_probs(logits + r * E, E, lane, pv);
    if (probs)
#pragma unroll
        for (int m = 0; m < kRouteLanesPer; ++m)
            if (lane + 64 * m < E) probs[r * E + lane + 64 * m] = pv[m];
    uint32_t taken = 0;  // bit m: expert lane + 64 m chosen
    double wtotal = 0.0;
    for (int64_t j = 0; j < K; ++j) {
        // the first untaken expert
        int64_t e0 = E;
#pragma unroll
        for (int m = kRouteLanesPer - 1; m >= 0; --m) {
            const bool open = lane + 64 * m < E && !((taken >> m) & 1u);
            const unsigned long long b = __ballot(open);
            if (b) e0 = 64 * m + (__ffsll(static_cast<long long>(b)) - 1);
        }
        const float p0 = wave_prob(pv, e0);
        int64_t best;
        if (p0 != p0) {
            best = e0;
        } else {
            float bv = -1.0f;  // below every probability (p >= +0)
            int64_t bi = E;
#pragma unroll
            for (int m = 0; m < kRouteLanesPer; ++m) {
                const int64_t e = lane + 64 * m;
                if (e < E && !((taken >> m) & 1u) && pv[m] > bv) {
                    bv = pv[m];
                    bi = e;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float ov = __shfl_xor(bv, off, 64);
                const int64_t oi = __shfl_xor(bi, off, 64);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            best = bi;
        }
        const float pb = wave_prob(pv, best);
        if (lane == static_cast<int>(best & 63)) taken |= 1u << (best >> 6);
        if (lane == 0) {
            indices[r * K + j] = best;
            weights[r * K + j] = pb;
        }
        wtotal += static_cast<double>(pb);
    }
    if (normalize && lane == 0)
        for (int64_t j = 0; j < K; ++j)
            weights[r * K + j] = static_cast<float>(static_cast<double>(weights[r * K + j]) / wtotal);
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

// moe_route_backward with one wave per row (E <= 256), the probabilities from wave_row_probs; the rank sums and
// the dot over e run serially in the reference's order, the per-expert terms one lane each.
__global__ __launch_bounds__(256) void moe_route_backward_wave_kernel(const float* __restrict__ logits,
                                                                      const int64_t* __restrict__ indices,
                                                                      const float* __restrict__ dweights,
                                                                      const float* __restrict__ dprob, int64_t rows,
                                                                      int64_t E, int64_t K, int normalize,
                                                                      float* __restrict__ dlogits) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float pv[kRouteLanesPer];
    wave_row_probs(logits + r * E, E, lane, pv);
    const int64_t* idx = indices + r * K;
    const float* dw = dweights + r * K;
    double total = 0.0, weighted = 0.0;
    for (int64_t j = 0; j < K; ++j) {
        const double p = static_cast<double>(wave_prob(pv, idx[j]));
        total += p;
        weighted += static_cast<double>(dw[j]) * p;
    }
    double dp[kRouteLanesPer], term[kRouteLanesPer];
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) {
        const int64_t e = lane + 64 * m;
        dp[m] = dprob && e < E ? static_cast<double>(dprob[r * E + e]) : 0.0;
    }
    for (int64_t j = 0; j < K; ++j) {
        const int64_t e = idx[j];
        const double d = static_cast<double>(dw[j]);
        const double add = normalize ? d / total - weighted / (total * total) : d;
#pragma unroll
        for (int m = 0; m < kRouteLanesPer; ++m)
            if (lane + 64 * m == e) dp[m] += add;
    }
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) term[m] = static_cast<double>(pv[m]) * dp[m];
    double dot = 0.0;
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) {
        if (64 * m >= E) break;
        const int n = E - 64 * m < 64 ? static_cast<int>(E - 64 * m) : 64;
        for (int k = 0; k < n; ++k) dot += readlane_f64(term[m], k);
    }
#pragma unroll
    for (int m = 0; m < kRouteLanesPer; ++m) {
        const int64_t e = lane + 64 * m;
        if (e < E) dlogits[r * E + e] = static_cast<float>(static_cast<double>(pv[m]) * (dp[m] - dot));
    }
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
        out[i] = addend ? acc + addend[i] : acc;
    }
}

// The same sums, one workgroup per row and 4 columns per thread (H % 4 == 0, 16-byte aligned rows): the row's
// choices are wave-uniform scalar loads, and the expert rows are read as 16-byte vectors.
__global__ __launch_bounds__(256) void moe_combine4_kernel(const float4* __restrict__ y,
                                                           const int64_t* __restrict__ order,
                                                           const int64_t* __restrict__ slot,
                                                           const float* __restrict__ weights,
                                                           const float4* __restrict__ addend, float4* __restrict__ out,
                                                           int64_t K, int64_t H4) {
    const int64_t r = blockIdx.x;
    for (int64_t d = threadIdx.x; d < H4; d += 256) {
        float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t k = 0; k < K; ++k) {
            const int64_t p = order[r * K + k];
            const float4 v = y[p * H4 + d];
            if (weights) {
                const float wk = weights[slot[p]];
                acc.x = acc.x + v.x * wk;
                acc.y = acc.y + v.y * wk;
                acc.z = acc.z + v.z * wk;
                acc.w = acc.w + v.w * wk;
            } else {
                acc.x = acc.x + v.x;
                acc.y = acc.y + v.y;
                acc.z = acc.z + v.z;
                acc.w = acc.w + v.w;
            }
        }
        if (addend) {
            const float4 a = addend[r * H4 + d];
            acc = float4{acc.x + a.x, acc.y + a.y, acc.z + a.z, acc.w + a.w};
        }
        out[r * H4 + d] = acc;
    }
}

// Per grouped position p (row r = row_of[p], routing slot q = slot[p]):
//   dweights[q] = f32(sum over d ascending of dout[r][d] y[p][d])   (dllm::dot, one lane per position)
//   dy[p][d]    = dout[r][d] * weights[q]
// A workgroup takes 64 positions; its four waves stage 64-column tiles of the products in LDS (writing dy on the
// way), then wave 0 runs the 64 chains. The tiles are double-buffered and the next tile's loads are in flight while
// wave 0 walks the current one: one barrier per tile.
__global__ __launch_bounds__(256) void moe_dweights_kernel(const float* __restrict__ dout, const float* __restrict__ y,
                                                           const int64_t* __restrict__ row_of,
                                                           const int64_t* __restrict__ slot,
                                                           const float* __restrict__ weights, int64_t positions,
                                                           int64_t H, float* __restrict__ dweights,
                                                           float* __restrict__ dy) {
    constexpr int kPer = 16;  // positions per wave
    __shared__ double prod[2][64][65];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t np = positions - p0 < 64 ? positions - p0 : 64;
    // this wave's positions: rows of dout, their routing weights (positions past the end repeat the last one)
    const float* grow[kPer];
    const float* yrow[kPer];
    float* dyrow[kPer];
    float wq[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int q = wave * kPer + k;
        const int64_t p = p0 + (q < np ? q : np - 1);
        grow[k] = dout + row_of[p] * H;
        yrow[k] = y + p * H;
        dyrow[k] = dy + p * H;
        wq[k] = weights[slot[p]];
    }
    float g[kPer], yv[kPer];
    auto load = [&](int64_t c0) {
        const int64_t c = c0 + lane < H ? c0 + lane : H - 1;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            g[k] = grow[k][c];
            yv[k] = yrow[k][c];
        }
    };
    load(0);
    double chain = 0.0;
    int buf = 0;
    for (int64_t c0 = 0; c0 < H; c0 += 64, buf ^= 1) {
        const int n = static_cast<int>(H - c0 < 64 ? H - c0 : 64);
        if (lane < n) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int q = wave * kPer + k;
                if (q < np) {
                    prod[buf][q][lane] = static_cast<double>(g[k]) * static_cast<double>(yv[k]);
                    dyrow[k][c0 + lane] = g[k] * wq[k];
                }
            }
        }
        __syncthreads();
        if (c0 + 64 < H) load(c0 + 64);
        if (wave == 0 && lane < np)
            for (int c = 0; c < n; ++c) chain += prod[buf][lane][c];
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

// ---- grouping the routed rows by expert on the device (backprop.py:308-357) ----
// The reference runs each expert over np.nonzero(indices == e): its rows ascending. Here the step's rows are grouped
// by expert (experts ascending, rows ascending inside an expert), which puts each window's rows of an expert in one
// contiguous run, and every quantity is an integer count or position, so the grouping is the same whatever order the
// threads run in:
//   moe_count_kernel   cnt[w][e]: rows of window w choosing expert e (integer atomics: order-free)
//   moe_starts_kernel  estart[e] (group starts), eseg[e][w] (window boundaries inside e's group), the router
//                      statistics' per-window counts += cnt
//   moe_place_kernel   one workgroup per expert walks the rows ascending; a row choosing e gets the next position
//                      (a block-wide prefix of the choosing rows): row_of[p], slot[p], pos_of[r K + j] = p
//   moe_order_kernel   order[r K + i] = the position of row r's i-th choice by ascending expert
__global__ __launch_bounds__(256) void moe_count_kernel(const int64_t* __restrict__ chosen, int64_t rows, int64_t K,
                                                        int64_t E, const int64_t* __restrict__ seg, int nseg,
                                                        unsigned long long* __restrict__ cnt, int* __restrict__ err) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < rows * K;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t e = chosen[i], r = i / K;
        if (e < 0 || e >= E) {
            *err = 1;
            continue;
        }
        int lo = 0, hi = nseg - 1;  // the window of row r: the last w with seg[w] <= r
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (seg[mid] <= r) lo = mid;
            else hi = mid - 1;
        }
        atomicAdd(&cnt[static_cast<int64_t>(lo) * E + e], 1ull);
    }
}

__global__ __launch_bounds__(256) void moe_starts_kernel(const unsigned long long* __restrict__ cnt, int64_t E, int nseg,
                                                         int64_t eseg_ld, int64_t* __restrict__ estart,
                                                         int64_t* __restrict__ eseg, int64_t* __restrict__ counts) {
    __shared__ int64_t total[1024];
    for (int64_t e = threadIdx.x; e < E; e += 256) {
        int64_t run = 0;
        eseg[e * eseg_ld] = 0;
        for (int w = 0; w < nseg; ++w) {
            const int64_t c = static_cast<int64_t>(cnt[static_cast<int64_t>(w) * E + e]);
            run += c;
            eseg[e * eseg_ld + w + 1] = run;
            counts[static_cast<int64_t>(w) * E + e] += c;
        }
        total[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t at = 0;
        for (int64_t e = 0; e < E; ++e) {
            estart[e] = at;
            at += total[e];
        }
        estart[E] = at;
    }
}

__global__ __launch_bounds__(256) void moe_place_kernel(const int64_t* __restrict__ chosen, int64_t rows, int64_t K,
                                                        const int64_t* __restrict__ estart,
                                                        int64_t* __restrict__ row_of, int64_t* __restrict__ slot,
                                                        int64_t* __restrict__ pos_of) {
    __shared__ int64_t wave_count[4];
    const int64_t e = blockIdx.x;
    const int lane = static_cast<int>(threadIdx.x) & 63, wave = static_cast<int>(threadIdx.x) >> 6;
    int64_t next = estart[e];  // the position the next choosing row takes
    for (int64_t r0 = 0; r0 < rows; r0 += 256) {
        const int64_t r = r0 + threadIdx.x;
        int64_t j = -1;
        if (r < rows)
            for (int64_t k = 0; k < K; ++k)
                if (chosen[r * K + k] == e) j = k;  // a row chooses an expert at most once
        const uint64_t mask = __ballot(j >= 0);
        const int64_t below = __popcll(mask & ((uint64_t{1} << lane) - 1));
        if (lane == 0) wave_count[wave] = __popcll(mask);
        __syncthreads();
        int64_t before = 0;
        for (int w = 0; w < wave; ++w) before += wave_count[w];
        if (j >= 0) {
            const int64_t p = next + before + below;
            row_of[p] = r;
            slot[p] = r * K + j;
            pos_of[r * K + j] = p;
        }
        next += wave_count[0] + wave_count[1] + wave_count[2] + wave_count[3];
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_order_kernel(const int64_t* __restrict__ chosen,
                                                        const int64_t* __restrict__ pos_of, int64_t rows, int64_t K,
                                                        int64_t* __restrict__ order) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= rows) return;
    // the row's choices by ascending expert: each output slot i takes the choice with exactly i smaller experts
    for (int64_t j = 0; j < K; ++j) {
        const int64_t e = chosen[r * K + j];
        int64_t rank = 0;
        for (int64_t k = 0; k < K; ++k) rank += chosen[r * K + k] < e ? 1 : 0;
        order[r * K + rank] = pos_of[r * K + j];
    }
}

__global__ __launch_bounds__(256) void zero_u64_kernel(unsigned long long* __restrict__ x, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
        x[i] = 0ull;
}

unsigned row_grid(int64_t rows) { return static_cast<unsigned>(ceil_div(static_cast<size_t>(rows), 256)); }

}  // namespace

int launch_moe_route(const float* logits, int64_t rows, int64_t experts, int64_t k, int normalize, int64_t* indices,
                     float* weights, float* probs, hipStream_t stream) {
    DLLM_REQUIRE(k >= 1 && k <= experts, "experts per token must be between 1 and the number of experts");
    if (rows == 0) return kOk;
    if (experts <= 64 * kRouteLanesPer)
        hipLaunchKernelGGL(moe_route_wave_kernel, dim3(static_cast<unsigned>(ceil_div(rows, 4))), dim3(256), 0, stream,
                           logits, rows, experts, k, normalize, indices, weights, probs);
    else
        hipLaunchKernelGGL(moe_route_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, logits, rows, experts, k,
                           normalize, indices, weights, probs);
    return check_launch("moe_route");
}

int launch_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights, const float* dprob,
                              int64_t rows, int64_t experts, int64_t k, int normalize, float* dlogits,
                              hipStream_t stream) {
    DLLM_REQUIRE(k >= 1 && k <= experts, "indices must be [rows, k] with k between 1 and the number of experts");
    if (rows == 0) return kOk;
    if (experts <= 64 * kRouteLanesPer)
        hipLaunchKernelGGL(moe_route_backward_wave_kernel, dim3(static_cast<unsigned>(ceil_div(rows, 4))), dim3(256),
                           0, stream, logits, indices, dweights, dprob, rows, experts, k, normalize, dlogits);
    else
        hipLaunchKernelGGL(moe_route_backward_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, logits, indices,
                           dweights, dprob, rows, experts, k, normalize, dlogits);
    return check_launch("moe_route_backward");
}

// The shared expert's gate (backprop.py:519-524), one 64-lane workgroup per row r: lane 0 forms the score
// f32(sum over k ascending of h2[r][k] w[k]) in double (linear with one output) and s[r] = f32(sigmoid(score));
// then term[r][d] = f32(y[r][d] s[r]). Without a gate (w null) term = y.
__global__ __launch_bounds__(64) void shared_gate_forward_kernel(const float* __restrict__ h2,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ y, float* __restrict__ s_out,
                                                                 float* __restrict__ term, int64_t H) {
    const int64_t r = blockIdx.x;
    __shared__ float sg;
    if (w == nullptr) {
        for (int64_t d = threadIdx.x; d < H; d += 64) term[r * H + d] = y[r * H + d];
        return;
    }
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int64_t k = 0; k < H; ++k) acc += static_cast<double>(h2[r * H + k]) * static_cast<double>(w[k]);
        sg = static_cast<float>(dsigmoid(static_cast<double>(static_cast<float>(acc))));
        s_out[r] = sg;
    }
    __syncthreads();
    for (int64_t d = threadIdx.x; d < H; d += 64) term[r * H + d] = y[r * H + d] * sg;
}

// Its backward (backprop.py:339-351), one 64-lane workgroup per row: dy[r][d] = f32(dmlp[r][d] s[r]) and
// dscore[r] = f32(f32(ds s) (1 - s)) with ds = dot(dmlp[r], y[r]) (dllm::dot: ascending, in double, rounded once).
__global__ __launch_bounds__(64) void shared_gate_backward_kernel(const float* __restrict__ dmlp,
                                                                  const float* __restrict__ y,
                                                                  const float* __restrict__ s,
                                                                  float* __restrict__ dy, float* __restrict__ dscore,
                                                                  int64_t H) {
    const int64_t r = blockIdx.x;
    const float sg = s[r];
    for (int64_t d = threadIdx.x; d < H; d += 64) dy[r * H + d] = dmlp[r * H + d] * sg;
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int64_t k = 0; k < H; ++k) acc += static_cast<double>(dmlp[r * H + k]) * static_cast<double>(y[r * H + k]);
        const float ds = static_cast<float>(acc);
        dscore[r] = (ds * sg) * (1.0f - sg);
    }
}

// The gate's input gradient added to dh (linear_backward with one output, then dh2 + dh2_gate):
// dh[r][k] = dh[r][k] + f32(dscore[r] w[k]) (the product of two floats is exact in double).
__global__ __launch_bounds__(256) void shared_gate_dx_kernel(const float* __restrict__ dscore,
                                                             const float* __restrict__ w, float* __restrict__ dh,
                                                             int64_t rows, int64_t H) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < rows * H;
         i += static_cast<int64_t>(gridDim.x) * 256)
        dh[i] = dh[i] + static_cast<float>(static_cast<double>(dscore[i / H]) * static_cast<double>(w[i % H]));
}

// The gate's weight gradient per window s: part[s][k] = f32(sum over the window's rows r ascending of
// dscore[r] h2[r][k]) in double (linear_backward's dw with one output).
__global__ __launch_bounds__(256) void shared_gate_dw_kernel(const float* __restrict__ dscore,
                                                             const float* __restrict__ h2,
                                                             const int64_t* __restrict__ seg, float* __restrict__ part,
                                                             int64_t H) {
    const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int w = blockIdx.y;
    if (k >= H) return;
    double acc = 0.0;
    for (int64_t r = seg[w]; r < seg[w + 1]; ++r)
        acc += static_cast<double>(dscore[r]) * static_cast<double>(h2[r * H + k]);
    part[static_cast<int64_t>(w) * H + k] = static_cast<float>(acc);
}

int launch_shared_gate_forward(const float* h2, const float* w, const float* y, float* s, float* term, int64_t rows,
                               int64_t H, hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(rows < (int64_t{1} << 31), "too many rows for the shared expert's gate");
    hipLaunchKernelGGL(shared_gate_forward_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, stream, h2, w, y,
                       s, term, H);
    return check_launch("shared gate");
}

int launch_shared_gate_backward(const float* dmlp, const float* y, const float* s, const float* w, const float* h2,
                                float* dy, float* dscore, float* dh, const int64_t* seg, int nseg, float* part,
                                int64_t rows, int64_t H, hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(rows < (int64_t{1} << 31), "too many rows for the shared expert's gate");
    if (dy) {  // null: dscore is already formed
        hipLaunchKernelGGL(shared_gate_backward_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, stream, dmlp,
                           y, s, dy, dscore, H);
        DLLM_TRY(check_launch("shared gate backward"));
    }
    if (dh) {
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(rows * H, 256), 16384));
        hipLaunchKernelGGL(shared_gate_dx_kernel, dim3(blocks), dim3(256), 0, stream, dscore, w, dh, rows, H);
        DLLM_TRY(check_launch("shared gate dx"));
    }
    if (part) {
        hipLaunchKernelGGL(shared_gate_dw_kernel, dim3(static_cast<unsigned>(ceil_div(H, 256)),
                                                       static_cast<unsigned>(nseg)),
                           dim3(256), 0, stream, dscore, h2, seg, part, H);
        DLLM_TRY(check_launch("shared gate dw"));
    }
    return kOk;
}

int launch_moe_combine(const float* y, const int64_t* order, const int64_t* slot, const float* weights,
                       const float* addend, float* out, int64_t rows, int64_t k, int64_t dim, hipStream_t stream) {
    const int64_t n = rows * dim;
    if (n == 0) return kOk;
    const bool vec = dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(addend) |
                                      reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec && rows < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(moe_combine4_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream,
                           reinterpret_cast<const float4*>(y), order, slot, weights,
                           reinterpret_cast<const float4*>(addend), reinterpret_cast<float4*>(out), k, dim / 4);
        return check_launch("moe_combine");
    }
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

int launch_moe_group_rows(const int64_t* chosen, int64_t rows, int64_t K, int64_t E, const int64_t* seg, int nseg,
                          void* cnt_scratch, int64_t* estart, int64_t* eseg, int64_t eseg_ld, int64_t* row_of,
                          int64_t* slot, int64_t* order, int64_t* pos_of, int64_t* counts, int* err,
                          hipStream_t stream) {
    DLLM_REQUIRE(E >= 1 && E <= 1024 && K >= 1 && K <= E && nseg >= 1, "grouping needs 1..1024 experts");
    if (rows == 0) return kOk;
    auto* cnt = static_cast<unsigned long long*>(cnt_scratch);
    const int64_t ncnt = static_cast<int64_t>(nseg) * E;
    hipLaunchKernelGGL(zero_u64_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(ncnt, 256), 1024))),
                       dim3(256), 0, stream, cnt, ncnt);
    hipLaunchKernelGGL(moe_count_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(rows * K, 256), 4096))),
                       dim3(256), 0, stream, chosen, rows, K, E, seg, nseg, cnt, err);
    hipLaunchKernelGGL(moe_starts_kernel, dim3(1), dim3(256), 0, stream, cnt, E, nseg, eseg_ld, estart, eseg, counts);
    hipLaunchKernelGGL(moe_place_kernel, dim3(static_cast<unsigned>(E)), dim3(256), 0, stream, chosen, rows, K, estart,
                       row_of, slot, pos_of);
    hipLaunchKernelGGL(moe_order_kernel, dim3(row_grid(rows)), dim3(256), 0, stream, chosen, pos_of, rows, K, order);
    return check_launch("moe grouping");
}

int launch_zero_i64(int64_t* x, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(zero_u64_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 256), 1024))),
                       dim3(256), 0, stream, reinterpret_cast<unsigned long long*>(x), n);
    return check_launch("zero");
}

}  // namespace dllm_hip
