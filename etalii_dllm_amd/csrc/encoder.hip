// Training kernels of the encoder and T5 families (cpp/include/dllm/grad.hpp:112-174, 300-389 and their forward
// passes, nn.hpp:412-432, 474-478, 827-856): exact GELU and its gradient, LayerNorm and its gradients, and T5's
// attention with an additive position bias and its gradients (dq, dk, dv, dbias).
//
// Every reduction keeps the reference's order and double accumulator:
// - GELU: elementwise, 0.5 x erfc(-x / sqrt 2) and its slope with the portable erf/erfc (devmath.h), rounded once.
// - LayerNorm: one lane per row runs the row's chains (sum, centred squares, sum of g = w dy and of g xhat) in index
//   order over columns staged in LDS; dw and db are one lane per column over the rows in order, xhat recomputed from
//   the row's saved mean and inv_std exactly as the row pass computes it.
// - Biased attention: one wave per (query t, head h). Scores are one lane per key (dot over head_dim ascending); the
//   maximum, the exponentials' total and D = sum p dp are one lane's scans over the keys in order; dq and the
//   forward's value sums are one lane per output column, keys ascending. dk[j, h] and dv[j, h] sum over queries t
//   ascending, one lane per output element, from the probabilities and ds saved per (t, h).
#include "attn_step.h"
#include "common.h"
#include "devmath.h"
#include "dllm_hip.h"
#include "kernels.h"
#include "lds_copy.h"

namespace dllm_hip {

namespace {

__global__ __launch_bounds__(256) void gelu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const double inv_sqrt2 = 7.07106781186547524401e-01;
    const double d = x[i];
    out[i] = static_cast<float>(0.5 * d * derfc(-d * inv_sqrt2));
}

__global__ __launch_bounds__(256) void gelu_backward_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                            float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const double inv_sqrt2 = 7.07106781186547524401e-01;
    const double inv_sqrt_2pi = 3.98942280401432677940e-01;
    const double d = x[i];
    const double slope = 0.5 * derfc(-d * inv_sqrt2) + d * dexp(-0.5 * d * d) * inv_sqrt_2pi;
    out[i] = static_cast<float>(static_cast<double>(dy[i]) * slope);
}

// LayerNorm rows: a 64-thread workgroup takes 16 rows. Each pass over the columns stages 64 columns of the 16 rows
// (and of dy, and the weights) in LDS with coalesced loads, the next chunk's loads in flight while lane r (r < 16)
// runs row r's chain over the staged columns in order. The chains are those of nn.hpp:412-426 and grad.hpp:112-163:
// total, then the centred squares, then (backward) the sums of g = w dy and of g xhat, each a double in index order.
constexpr int kLnRows = 16;

template <bool kBackward>
struct LnTiles {
    float x[kLnRows][65];
    float dy[kBackward ? kLnRows : 1][65];
    float w[64];
    float b[64];
};

template <bool kBackward>
struct LnChunk {
    float x[kLnRows];
    float dy[kBackward ? kLnRows : 1];
    float w, b;
};

template <bool kBackward>
__device__ inline void ln_fetch(LnChunk<kBackward>& c, const float* x, const float* dy, const float* w,
                                const float* b, int64_t r0, int64_t c0, int64_t rows, int64_t dim, int lane) {
    const int64_t col = c0 + lane;
    const bool in_col = col < dim;
    for (int rr = 0; rr < kLnRows; ++rr) {
        const bool ok = in_col && r0 + rr < rows;
        c.x[rr] = ok ? x[(r0 + rr) * dim + col] : 0.0f;
        if constexpr (kBackward) c.dy[rr] = ok ? dy[(r0 + rr) * dim + col] : 0.0f;
    }
    c.w = in_col ? w[col] : 0.0f;
    c.b = (in_col && b) ? b[col] : 0.0f;
}

template <bool kBackward>
__device__ inline void ln_stage(LnTiles<kBackward>& t, const LnChunk<kBackward>& c, int lane) {
    for (int rr = 0; rr < kLnRows; ++rr) {
        t.x[rr][lane] = c.x[rr];
        if constexpr (kBackward) t.dy[rr][lane] = c.dy[rr];
    }
    t.w[lane] = c.w;
    t.b[lane] = c.b;
}

// One pass over the columns: body(c0, n) runs on lanes 0..15 with chunk [c0, c0 + n) staged; after(c0, n) runs on
// all lanes once body is done (a store of the chunk's results).
template <bool kBackward, typename Body, typename After>
__device__ inline void ln_pass(LnTiles<kBackward>& t, const float* x, const float* dy, const float* w, const float* b,
                               int64_t r0, int64_t rows, int64_t dim, int lane, Body body, After after) {
    LnChunk<kBackward> c;
    ln_fetch<kBackward>(c, x, dy, w, b, r0, 0, rows, dim, lane);
    for (int64_t c0 = 0; c0 < dim; c0 += 64) {
        lds_barrier();
        ln_stage<kBackward>(t, c, lane);
        lds_barrier();
        if (c0 + 64 < dim) ln_fetch<kBackward>(c, x, dy, w, b, r0, c0 + 64, rows, dim, lane);
        const int n = dim - c0 < 64 ? static_cast<int>(dim - c0) : 64;
        if (lane < kLnRows) body(c0, n);
        lds_barrier();
        after(c0, n);
    }
}

// mean and inv_std of the workgroup's rows (lane r holds row r's); two passes.
template <bool kBackward>
__device__ inline void ln_moments(LnTiles<kBackward>& t, const float* x, const float* dy, const float* w,
                                  int64_t r0, int64_t rows, int64_t dim, double eps, int lane, double* mean_out,
                                  double* inv_out) {
    double total = 0.0;
    ln_pass<kBackward>(
        t, x, dy, w, nullptr, r0, rows, dim, lane,
        [&](int64_t, int n) {
            for (int j = 0; j < n; ++j) total += static_cast<double>(t.x[lane][j]);
        },
        [](int64_t, int) {});
    const double mean = total / static_cast<double>(dim);
    double sum_sq = 0.0;
    ln_pass<kBackward>(
        t, x, dy, w, nullptr, r0, rows, dim, lane,
        [&](int64_t, int n) {
            for (int j = 0; j < n; ++j) {
                const double c = static_cast<double>(t.x[lane][j]) - mean;
                sum_sq += c * c;
            }
        },
        [](int64_t, int) {});
    *mean_out = mean;
    *inv_out = 1.0 / sqrt(sum_sq / static_cast<double>(dim) + eps);
}

// the chunk's results, written by lanes 0..15 into t.x, stored by all lanes with coalesced writes
template <bool kBackward>
__device__ inline void ln_store(const LnTiles<kBackward>& t, float* out, int64_t r0, int64_t c0, int n, int64_t rows,
                                int64_t dim, int lane) {
    if (lane >= n) return;
    for (int rr = 0; rr < kLnRows; ++rr)
        if (r0 + rr < rows) out[(r0 + rr) * dim + c0 + lane] = t.x[rr][lane];
}

__global__ __launch_bounds__(64) void layer_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ b, float* __restrict__ out,
                                                        int64_t rows, int64_t dim, double eps) {
    __shared__ LnTiles<false> t;
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kLnRows;
    double mean = 0.0, inv_std = 0.0;
    ln_moments<false>(t, x, nullptr, w, r0, rows, dim, eps, lane, &mean, &inv_std);
    ln_pass<false>(
        t, x, nullptr, w, b, r0, rows, dim, lane,
        [&](int64_t, int n) {
            for (int j = 0; j < n; ++j) {
                const double scaled = (static_cast<double>(t.x[lane][j]) - mean) * inv_std *
                                      static_cast<double>(t.w[j]);
                t.x[lane][j] = static_cast<float>(scaled + static_cast<double>(t.b[j]));
            }
        },
        [&](int64_t c0, int n) { ln_store<false>(t, out, r0, c0, n, rows, dim, lane); });
}

// grad.hpp:112-163, the row part: dx, and each row's mean and inv_std for the column sums.
__global__ __launch_bounds__(64) void layer_norm_backward_rows_kernel(const float* __restrict__ x,
                                                                      const float* __restrict__ w,
                                                                      const float* __restrict__ dy,
                                                                      float* __restrict__ dx,
                                                                      double* __restrict__ stats, int64_t rows,
                                                                      int64_t dim, double eps) {
    __shared__ LnTiles<true> t;
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kLnRows;
    double mean = 0.0, inv_std = 0.0;
    ln_moments<true>(t, x, dy, w, r0, rows, dim, eps, lane, &mean, &inv_std);
    if (lane < kLnRows && r0 + lane < rows) {
        stats[2 * (r0 + lane)] = mean;
        stats[2 * (r0 + lane) + 1] = inv_std;
    }
    if (!dx) return;
    double g_sum = 0.0, gx_sum = 0.0;
    ln_pass<true>(
        t, x, dy, w, nullptr, r0, rows, dim, lane,
        [&](int64_t, int n) {
            for (int j = 0; j < n; ++j) {
                const double xhat = (static_cast<double>(t.x[lane][j]) - mean) * inv_std;
                const double g = static_cast<double>(t.w[j]) * static_cast<double>(t.dy[lane][j]);
                g_sum += g;
                gx_sum += g * xhat;
            }
        },
        [](int64_t, int) {});
    const double g_mean = g_sum / static_cast<double>(dim);
    const double gx_mean = gx_sum / static_cast<double>(dim);
    ln_pass<true>(
        t, x, dy, w, nullptr, r0, rows, dim, lane,
        [&](int64_t, int n) {
            for (int j = 0; j < n; ++j) {
                const double xhat = (static_cast<double>(t.x[lane][j]) - mean) * inv_std;
                const double g = static_cast<double>(t.w[j]) * static_cast<double>(t.dy[lane][j]);
                t.x[lane][j] = static_cast<float>(inv_std * (g - g_mean - xhat * gx_mean));
            }
        },
        [&](int64_t c0, int n) { ln_store<true>(t, dx, r0, c0, n, rows, dim, lane); });
}

// The column part: dw_i = sum over rows ascending of dy xhat, db_i = sum of dy. A chain has one term per row, so the
// kernel is bound by how many rows' loads are in flight: a 1024-thread workgroup takes 16 columns, thread t holds row
// slot t / 16 of each 64-row chunk for column t % 16, with kLnColDepth chunks loaded ahead in registers. Each
// chunk's terms dy xhat (double) and dy go to LDS, and lanes 0-15 of wave 0 add the previous chunk's onto the chains
// in row order; two LDS buffers.
constexpr int kLnColRows = 64;
constexpr int kLnColWidth = 16;
constexpr int kLnColDepth = 8;

__global__ __launch_bounds__(1024) void layer_norm_backward_cols_kernel(const float* __restrict__ x,
                                                                        const float* __restrict__ dy,
                                                                        const double* __restrict__ stats,
                                                                        float* __restrict__ dw, float* __restrict__ db,
                                                                        int64_t rows, int64_t dim) {
    __shared__ double terms[2][kLnColRows][kLnColWidth];
    __shared__ float dys[2][kLnColRows][kLnColWidth];
    const int tid = static_cast<int>(threadIdx.x);
    const int c16 = tid % kLnColWidth, slot = tid / kLnColWidth;
    const int64_t col = static_cast<int64_t>(blockIdx.x) * kLnColWidth + c16;
    const bool in_col = col < dim;
    const int64_t chunks = (rows + kLnColRows - 1) / kLnColRows;
    double dw_acc = 0.0, db_acc = 0.0;
    float xv[kLnColDepth], dv[kLnColDepth];
    double mv[kLnColDepth], sv[kLnColDepth];
    // loads at clamped addresses, unconditionally (the counter waits then cover exactly the older slots); terms of
    // rows or columns past the end are formed but never added or stored
    const int64_t col_c = in_col ? col : dim - 1;
    const auto fetch = [&](int64_t c, int k) {
        const int64_t r = c * kLnColRows + slot < rows ? c * kLnColRows + slot : rows - 1;
        xv[k] = x[r * dim + col_c];
        dv[k] = dy[r * dim + col_c];
        mv[k] = stats[2 * r];
        sv[k] = stats[2 * r + 1];
    };
#pragma unroll
    for (int k = 0; k < kLnColDepth; ++k) fetch(k < chunks ? k : chunks - 1, k);
    for (int64_t c0 = 0; c0 <= chunks; c0 += kLnColDepth) {
#pragma unroll
        for (int k = 0; k < kLnColDepth; ++k) {
            const int64_t c = c0 + k;
            if (c > chunks) break;
            const int buf = static_cast<int>(c & 1);
            const double xhat = (static_cast<double>(xv[k]) - mv[k]) * sv[k];
            terms[buf][slot][c16] = static_cast<double>(dv[k]) * xhat;
            dys[buf][slot][c16] = dv[k];
            fetch(c + kLnColDepth < chunks ? c + kLnColDepth : chunks - 1, k);
            if (c > 0 && tid < kLnColWidth) {
                const int pbuf = buf ^ 1;
                const int64_t r0 = (c - 1) * kLnColRows;
                const int n = rows - r0 < kLnColRows ? static_cast<int>(rows - r0) : kLnColRows;
                // straight-line (no inner loop, so the compiler's load-counter waits stay exact); rows past the
                // end are skipped by selects
#pragma unroll
                for (int rr = 0; rr < kLnColRows; ++rr) {
                    const double t = dw_acc + terms[pbuf][rr][tid];
                    const double d = db_acc + static_cast<double>(dys[pbuf][rr][tid]);
                    dw_acc = rr < n ? t : dw_acc;
                    db_acc = rr < n ? d : db_acc;
                }
            }
            lds_barrier();
        }
    }
    if (tid < kLnColWidth && in_col) {
        if (dw) dw[col] = static_cast<float>(dw_acc);
        if (db) db[col] = static_cast<float>(db_acc);
    }
}

// The same column sums with the raw chunks copied straight to LDS (global_load_lds_dwordx4) kLnColRing chunks
// ahead, so the copies in flight are tracked by explicit counter waits rather than by registers (dim % 4 == 0 and
// 16-byte aligned x, dy). Waves 0-3 copy x (16 rows each, 4 lanes per row), waves 4-7 dy, wave 8 the rows' (mean,
// inv_std): one copy per wave per chunk, so "at most kLnColRing - 2 newer copies pending" means this chunk landed.
constexpr int kLnColRing = 8;

struct LnColSlot {
    float x[kLnColRows][kLnColWidth];
    float dy[kLnColRows][kLnColWidth];
    double st[kLnColRows][2];
};

__global__ __launch_bounds__(1024) void layer_norm_backward_cols_lds_kernel(const float* __restrict__ x,
                                                                            const float* __restrict__ dy,
                                                                            const double* __restrict__ stats,
                                                                            float* __restrict__ dw,
                                                                            float* __restrict__ db, int64_t rows,
                                                                            int64_t dim) {
    __shared__ __align__(16) LnColSlot ring[kLnColRing];
    // [buffer][row][column]: dy xhat in columns 0-15, f64(dy) in 16-31 (lane l < 32 runs chain l)
    __shared__ double terms[2][kLnColRows][2 * kLnColWidth];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int c16 = tid % kLnColWidth, slot = tid / kLnColWidth;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kLnColWidth;
    const int64_t chunks = (rows + kLnColRows - 1) / kLnColRows;
    // this wave's copy: row (clamped) and 4-column group (clamped) of the chunk
    const auto issue = [&](int64_t c) {
        if (wave > 8) return;
        const int64_t cc = c < chunks ? c : chunks - 1;
        LnColSlot& dst = ring[cc % kLnColRing];
        if (wave < 8) {
            const int rr = 16 * (wave & 3) + lane / 4;
            const int64_t r = cc * kLnColRows + rr < rows ? cc * kLnColRows + rr : rows - 1;
            const int64_t g = col0 + 4 * (lane & 3) < dim ? col0 + 4 * (lane & 3) : dim - 4;
            const float* src = (wave < 4 ? x : dy) + r * dim + g;
            copy16_to_lds(src, wave < 4 ? &dst.x[16 * (wave & 3)][0] : &dst.dy[16 * (wave & 3)][0]);
        } else {
            const int64_t r = cc * kLnColRows + lane < rows ? cc * kLnColRows + lane : rows - 1;
            copy16_to_lds(stats + 2 * r, &dst.st[0][0]);
        }
    };
    for (int k = 0; k < kLnColRing - 1; ++k) issue(k);
    double acc = 0.0;  // lane l < 16: dw of column l; 16 <= l < 32: db of column l - 16
    for (int64_t c = 0; c <= chunks; ++c) {
        // chunk c landed (kLnColRing - 2 newer copies may be pending), the previous chunk's terms are written, and
        // every wave is done reading the ring slot the next copy refills
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kLnColRing - 2) : "memory");
        issue(c + kLnColRing - 1);
        const LnColSlot& src = ring[(c < chunks ? c : chunks - 1) % kLnColRing];
        const double xhat = (static_cast<double>(src.x[slot][c16]) - src.st[slot][0]) * src.st[slot][1];
        const int buf = static_cast<int>(c & 1);
        terms[buf][slot][c16] = static_cast<double>(src.dy[slot][c16]) * xhat;
        terms[buf][slot][kLnColWidth + c16] = static_cast<double>(src.dy[slot][c16]);
        if (c > 0 && tid < 2 * kLnColWidth) {
            const int pbuf = buf ^ 1;
            const int64_t r0 = (c - 1) * kLnColRows;
            const int n = rows - r0 < kLnColRows ? static_cast<int>(rows - r0) : kLnColRows;
            if (n == kLnColRows) {
#pragma unroll
                for (int rr = 0; rr < kLnColRows; ++rr) acc += terms[pbuf][rr][tid];
            } else {
                for (int rr = 0; rr < n; ++rr) acc += terms[pbuf][rr][tid];
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the end drain before exit
    if (tid < kLnColWidth && col0 + tid < dim && dw) dw[col0 + tid] = static_cast<float>(acc);
    if (tid >= kLnColWidth && tid < 2 * kLnColWidth && col0 + tid - kLnColWidth < dim && db)
        db[col0 + tid - kLnColWidth] = static_cast<float>(acc);
}

struct BiasedShape {
    int64_t q_len, kv_len, heads, hd, vd;
    double scale;
};

// Scores s_j = (q . k_j + bias) scale, then e_j = exp(s_j - max) into e[0 .. kv_len), and returns 1 / total with
// total the serial sum of e over j ascending (lane 0's chain, broadcast through LDS).
__device__ inline double biased_probabilities(const float* qh, const float* k, const float* bh, const BiasedShape& s,
                                              int64_t h, double* e, double* shared, int lane) {
    for (int64_t j = lane; j < s.kv_len; j += 64) {
        const float* kj = k + (j * s.heads + h) * s.hd;
        double d = 0.0;
        for (int64_t i = 0; i < s.hd; ++i) d += static_cast<double>(qh[i]) * static_cast<double>(kj[i]);
        e[j] = (d + static_cast<double>(bh[j])) * s.scale;
    }
    __syncthreads();
    if (lane == 0) {  // the maximum as the reference's scan takes it (keys in order; a NaN first key stays)
        double m = e[0];
        for (int64_t j = 1; j < s.kv_len; ++j)
            if (e[j] > m) m = e[j];
        shared[0] = m;
    }
    __syncthreads();
    const double max = shared[0];
    for (int64_t j = lane; j < s.kv_len; j += 64) e[j] = dexp(e[j] - max);
    __syncthreads();
    if (lane == 0) {
        double total = 0.0;
        for (int64_t j = 0; j < s.kv_len; ++j) total += e[j];
        shared[1] = 1.0 / total;
    }
    __syncthreads();
    return shared[1];
}

// nn.hpp:827-856: out = f32((sum_j e_j v_j) (1 / total)); one 64-thread workgroup per (t, h).
__global__ __launch_bounds__(64) void biased_attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                              const float* __restrict__ v,
                                                              const float* __restrict__ bias, float* __restrict__ out,
                                                              double* __restrict__ scratch, BiasedShape s) {
    __shared__ double shared[2];
    const int64_t row = blockIdx.x;  // t * heads + h
    const int64_t t = row / s.heads, h = row % s.heads;
    const int lane = static_cast<int>(threadIdx.x);
    float* oh = out + row * s.vd;
    if (s.kv_len == 0) {
        for (int64_t i = lane; i < s.vd; i += 64) oh[i] = 0.0f;
        return;
    }
    double* e = scratch + row * s.kv_len;
    const double inv = biased_probabilities(q + row * s.hd, k, bias + (h * s.q_len + t) * s.kv_len, s, h, e, shared,
                                            lane);
    for (int64_t i = lane; i < s.vd; i += 64) {
        double acc = 0.0;
        for (int64_t j = 0; j < s.kv_len; ++j) acc += e[j] * static_cast<double>(v[(j * s.heads + h) * s.vd + i]);
        oh[i] = static_cast<float>(acc * inv);
    }
}

// grad.hpp:300-389, the (t, h) part: p, dp, D, ds (dbias), dq; p and ds saved for dk and dv.
__global__ __launch_bounds__(64) void biased_attention_backward_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ bias, const float* __restrict__ dout, float* __restrict__ dq,
    float* __restrict__ dbias, double* __restrict__ p_save, double* __restrict__ ds_save, BiasedShape s) {
    __shared__ double shared[2];
    const int64_t row = blockIdx.x;
    const int64_t t = row / s.heads, h = row % s.heads;
    const int lane = static_cast<int>(threadIdx.x);
    float* dqh = dq + row * s.hd;
    if (s.kv_len == 0) {
        for (int64_t i = lane; i < s.hd; i += 64) dqh[i] = 0.0f;
        return;
    }
    const float* qh = q + row * s.hd;
    const float* doh = dout + row * s.vd;
    double* p = p_save + row * s.kv_len;
    double* ds = ds_save + row * s.kv_len;
    const double inv = biased_probabilities(qh, k, bias + (h * s.q_len + t) * s.kv_len, s, h, p, shared, lane);
    for (int64_t j = lane; j < s.kv_len; j += 64) {
        p[j] = p[j] * inv;
        const float* vj = v + (j * s.heads + h) * s.vd;
        double d = 0.0;
        for (int64_t i = 0; i < s.vd; ++i) d += static_cast<double>(doh[i]) * static_cast<double>(vj[i]);
        ds[j] = d;  // dp for now
    }
    __syncthreads();
    if (lane == 0) {
        double weighted = 0.0;
        for (int64_t j = 0; j < s.kv_len; ++j) weighted += p[j] * ds[j];
        shared[0] = weighted;
    }
    __syncthreads();
    const double weighted = shared[0];
    float* dbh = dbias + (h * s.q_len + t) * s.kv_len;
    for (int64_t j = lane; j < s.kv_len; j += 64) {
        const double g = p[j] * (ds[j] - weighted) * s.scale;
        ds[j] = g;
        dbh[j] = static_cast<float>(g);
    }
    __syncthreads();
    for (int64_t i = lane; i < s.hd; i += 64) {
        double acc = 0.0;
        for (int64_t j = 0; j < s.kv_len; ++j) acc += ds[j] * static_cast<double>(k[(j * s.heads + h) * s.hd + i]);
        dqh[i] = static_cast<float>(acc);
    }
}

// dk[j][h][i] = sum over t ascending of ds[t, h][j] q[t][h][i]; dv likewise with p and dout.
__global__ __launch_bounds__(256) void biased_attention_backward_kv_kernel(
    const float* __restrict__ q, const float* __restrict__ dout, const double* __restrict__ p_save,
    const double* __restrict__ ds_save, float* __restrict__ dk, float* __restrict__ dv, BiasedShape s) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t nk = s.kv_len * s.heads * s.hd, nv = s.kv_len * s.heads * s.vd;
    if (e < nk) {
        const int64_t i = e % s.hd, jh = e / s.hd, h = jh % s.heads, j = jh / s.heads;
        double acc = 0.0;
        for (int64_t t = 0; t < s.q_len; ++t) {
            const int64_t row = t * s.heads + h;
            acc += ds_save[row * s.kv_len + j] * static_cast<double>(q[row * s.hd + i]);
        }
        dk[e] = static_cast<float>(acc);
    } else if (e < nk + nv) {
        const int64_t f = e - nk;
        const int64_t i = f % s.vd, jh = f / s.vd, h = jh % s.heads, j = jh / s.heads;
        double acc = 0.0;
        for (int64_t t = 0; t < s.q_len; ++t) {
            const int64_t row = t * s.heads + h;
            acc += p_save[row * s.kv_len + j] * static_cast<double>(dout[row * s.vd + i]);
        }
        dv[f] = static_cast<float>(acc);
    }
}

// biased_attention_weights (interp.hpp:79-121) on the per-(query, head) path: f32(e_j (1 / total)).
__global__ __launch_bounds__(64) void biased_weights_rows_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ bias,
                                                                 float* __restrict__ out, double* __restrict__ scratch,
                                                                 BiasedShape s) {
    __shared__ double shared[2];
    const int64_t row = blockIdx.x;
    const int64_t t = row / s.heads, h = row % s.heads;
    const int lane = static_cast<int>(threadIdx.x);
    double* e = scratch + row * s.kv_len;
    const double inv = biased_probabilities(q + row * s.hd, k, bias + (h * s.q_len + t) * s.kv_len, s, h, e, shared,
                                            lane);
    for (int64_t j = lane; j < s.kv_len; j += 64) out[row * s.kv_len + j] = static_cast<float>(e[j] * inv);
}

// ---- the matrix-core path for self-attention shapes (q_len == kv_len = n, head_dim and value_dim multiples of 4) --
// Per head, as the training step's attention lays it out: S^T[j][t] = sum_i k[j][i] q[t][i] (FP64 matrix cores,
// exact products), then s = (S^T + bias[h][t][j]) scale, the softmax chains per query over every key, and the value,
// dq, dk and dv sums as multiply-then-add tiles over keys (or queries) ascending: the reference's orders.

__global__ void biased_seg_kernel(int64_t* seg, int64_t n) {
    if (threadIdx.x == 0) {
        seg[0] = 0;
        seg[1] = n;
    }
}

// et[h][j][t] = (et[h][j][t] + bias[h][t][j]) scale for j, t < n; a 64 x 64 tile through LDS so the bias is read
// along j and the scores along t.
__global__ __launch_bounds__(256) void biased_scores_kernel(double* __restrict__ et, const float* __restrict__ bias,
                                                            int64_t n, int64_t Tp, double scale) {
    __shared__ float tile[64][65];
    const int64_t h = blockIdx.z;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64, j0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const float* bh = bias + h * n * n;
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, j = j0 + tx;
        tile[k][tx] = (t < n && j < n) ? bh[t * n + j] : 0.0f;
    }
    __syncthreads();
    double* eh = et + h * Tp * Tp;
    for (int k = ty; k < 64; k += 4) {
        const int64_t j = j0 + k, t = t0 + tx;
        if (j < n && t < n) eh[j * Tp + t] = (eh[j * Tp + t] + static_cast<double>(tile[tx][k])) * scale;
    }
}

// out[t][h][j] = f32(e[h][j][t] inv[h][t]) (biased_attention_weights), transposed through LDS.
__global__ __launch_bounds__(256) void biased_weights_kernel(const double* __restrict__ et,
                                                             const double* __restrict__ inv, float* __restrict__ out,
                                                             int64_t n, int64_t Tp, int64_t heads) {
    __shared__ float tile[64][65];
    const int64_t h = blockIdx.z;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64, j0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const double* eh = et + h * Tp * Tp;
    const double iv = t0 + tx < n ? inv[h * Tp + t0 + tx] : 0.0;
    for (int k = ty; k < 64; k += 4) {
        const int64_t j = j0 + k, t = t0 + tx;
        tile[k][tx] = (j < n && t < n) ? static_cast<float>(eh[j * Tp + t] * iv) : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, j = j0 + tx;
        if (t < n && j < n) out[(t * heads + h) * n + j] = tile[tx][k];
    }
}

// dbias[h][t][j] = f32(ds[h][t][j]) from the key-row layout the softmax backward writes.
__global__ __launch_bounds__(256) void biased_dbias_kernel(const double* __restrict__ dsg, float* __restrict__ dbias,
                                                           int64_t n, int64_t Tp) {
    const int64_t h = blockIdx.z, t = blockIdx.y;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (j < n) dbias[(h * n + t) * n + j] = static_cast<float>(dsg[h * Tp * Tp + t * Tp + j]);
}

unsigned blocks_for(int64_t n, int per) { return static_cast<unsigned>(ceil_div(static_cast<size_t>(n), per)); }


// Workspace of the matrix-core path: [seg | q^T | E^T | inv] for the forward and the weights, then
// [dout^T | dP^T | D | p | ds] for the backward.
struct BiasedLayout {
    int64_t n = 0, Tp = 0, heads = 0, hd = 0, vd = 0;
    size_t seg = 0, qt = 0, et = 0, inv = 0, forward = 0;
    size_t dot = 0, dpt = 0, dvec = 0, pg = 0, dsg = 0, backward = 0;
};

bool biased_fast(size_t q_len, size_t kv_len, size_t heads, size_t hd, size_t vd) {
    return q_len == kv_len && q_len > 0 && q_len <= 65535 && heads > 0 && hd > 0 && vd > 0 && hd % 4 == 0 &&
           vd % 4 == 0;
}

BiasedLayout biased_layout(size_t n, size_t heads, size_t hd, size_t vd) {
    BiasedLayout L;
    L.n = static_cast<int64_t>(n);
    L.Tp = static_cast<int64_t>(round_up(n, 64));
    L.heads = static_cast<int64_t>(heads);
    L.hd = static_cast<int64_t>(hd);
    L.vd = static_cast<int64_t>(vd);
    const size_t Tp = static_cast<size_t>(L.Tp), sq = heads * Tp * Tp * sizeof(double);
    size_t off = 0;
    const auto take = [&](size_t bytes) {
        const size_t at = off;
        off += round_up(bytes, 256);
        return at;
    };
    L.seg = take(2 * sizeof(int64_t));
    L.qt = take(heads * hd * Tp * sizeof(float));
    L.et = take(sq);
    L.inv = take(heads * Tp * sizeof(double));
    L.forward = off;
    L.dot = take(heads * vd * Tp * sizeof(float));
    L.dpt = take(sq);
    L.dvec = take(heads * Tp * sizeof(double));
    L.pg = take(sq);
    L.dsg = take(sq);
    L.backward = off;
    return L;
}

template <typename T>
T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

AttnTileCall biased_call(const BiasedLayout& L, const int64_t* seg) {
    AttnTileCall c;
    c.seg = seg;
    c.windows = 1;
    c.heads = L.heads;
    c.max_len = L.n;
    c.group = 1;
    c.window = 0;
    c.mask = kMaskNone;
    return c;
}

// rows of one head in a [length][heads][dim] tensor
AttnOperand head_rows(const float* p, int64_t heads, int64_t dim) {
    return AttnOperand{p, 0, heads * dim, dim, 1, heads * dim, 0, 1};
}

// [head][Tp][Tp] or [head][dim][Tp] blocks
AttnOperand head_block(const void* p, int64_t rows, int64_t Tp, int64_t heads) {
    return AttnOperand{p, heads * rows * Tp, 0, rows * Tp, 1, Tp, 0, 1};
}

// S^T, the biased scores, E^T and inv of every head (the forward's probabilities)
int biased_probabilities_fast(const float* q, const float* k, const float* bias, const BiasedLayout& L, double scale,
                              void* ws, hipStream_t s) {
    int64_t* seg = at<int64_t>(ws, L.seg);
    float* qt = at<float>(ws, L.qt);
    double* et = at<double>(ws, L.et);
    hipLaunchKernelGGL(biased_seg_kernel, dim3(1), dim3(64), 0, s, seg, L.n);
    DLLM_TRY(launch_heads_transpose(q, L.heads * L.hd, L.hd, qt, false, L.Tp, L.hd * L.Tp, seg, 1, L.heads, L.n, s));
    AttnTileCall g = biased_call(L, seg);
    g.A = head_rows(k, L.heads, L.hd);
    g.a_float = true;
    g.a_row_alloc = L.hd;
    g.B = head_block(qt, L.hd, L.Tp, L.heads);
    g.C = head_block(et, L.Tp, L.Tp, L.heads);
    g.head_dim = L.hd;
    g.rows_kind = 0;
    g.cols_kind = 0;
    g.L = L.hd;
    g.cols_per_lane = 4;
    g.b_row_alloc = L.Tp;
    g.exact_products = true;
    g.out_double = true;
    g.out_scale = 1.0;
    DLLM_TRY(launch_attn_tiles(g, s));
    const unsigned tiles = static_cast<unsigned>(ceil_div(static_cast<size_t>(L.n), 64));
    hipLaunchKernelGGL(biased_scores_kernel, dim3(tiles, tiles, static_cast<unsigned>(L.heads)), dim3(256), 0, s, et,
                       bias, L.n, L.Tp, scale);
    DLLM_TRY(check_launch("biased scores"));
    return launch_softmax_rows(et, L.Tp, L.Tp * L.Tp, seg, 1, L.heads, L.n, kAllKeys, at<double>(ws, L.inv), L.Tp, s);
}

// C[i] = sum over l < n ascending of A[l][i] B[l] (multiply, then add), float output, optional row scale
AttnTileCall biased_sum(const BiasedLayout& L, const int64_t* seg, const double* A, const float* B, int64_t b_dim,
                        float* C, const double* rowscale) {
    AttnTileCall c = biased_call(L, seg);
    c.A = head_block(A, L.Tp, L.Tp, L.heads);
    c.B = head_rows(B, L.heads, b_dim);
    c.C = head_rows(C, L.heads, b_dim);
    c.head_dim = b_dim;
    c.rows_kind = 0;
    c.cols_kind = 1;
    c.L = L.n;
    c.cols_per_lane = b_dim > 64 ? 2 : 1;
    c.exact_products = false;
    c.out_double = false;
    c.rowscale = rowscale;
    c.rowscale_zstride = rowscale ? L.Tp : 0;
    return c;
}

int biased_forward_fast(const float* q, const float* k, const float* v, const float* bias, float* out,
                        const BiasedLayout& L, double scale, void* ws, hipStream_t s) {
    DLLM_TRY(biased_probabilities_fast(q, k, bias, L, scale, ws, s));
    return launch_attn_tiles(biased_sum(L, at<int64_t>(ws, L.seg), at<double>(ws, L.et), v, L.vd, out,
                                        at<double>(ws, L.inv)),
                             s);
}

int biased_backward_fast(const float* q, const float* k, const float* v, const float* bias, const float* dout,
                         float* dq, float* dk, float* dv, float* dbias, const BiasedLayout& L, double scale, void* ws,
                         hipStream_t s) {
    DLLM_TRY(biased_probabilities_fast(q, k, bias, L, scale, ws, s));
    const int64_t* seg = at<int64_t>(ws, L.seg);
    double* et = at<double>(ws, L.et);
    double* dpt = at<double>(ws, L.dpt);
    double* pg = at<double>(ws, L.pg);
    double* dsg = at<double>(ws, L.dsg);
    float* dot = at<float>(ws, L.dot);
    DLLM_TRY(launch_heads_transpose(dout, L.heads * L.vd, L.vd, dot, false, L.Tp, L.vd * L.Tp, seg, 1, L.heads, L.n,
                                    s));
    // dP^T[j][t] = sum_i v[j][i] dout[t][i]
    AttnTileCall g = biased_call(L, seg);
    g.A = head_rows(v, L.heads, L.vd);
    g.a_float = true;
    g.a_row_alloc = L.vd;
    g.B = head_block(dot, L.vd, L.Tp, L.heads);
    g.C = head_block(dpt, L.Tp, L.Tp, L.heads);
    g.head_dim = L.vd;
    g.rows_kind = 0;
    g.cols_kind = 0;
    g.L = L.vd;
    g.cols_per_lane = 4;
    g.b_row_alloc = L.Tp;
    g.exact_products = true;
    g.out_double = true;
    g.out_scale = 1.0;
    DLLM_TRY(launch_attn_tiles(g, s));
    // D, p = e inv, ds = p (dp - D) scale: ds over dP^T, p and ds as [h][t][j]
    DLLM_TRY(launch_dsoftmax_regroup(et, dpt, L.Tp, L.Tp * L.Tp, seg, 1, L.heads, 1, L.n, kAllKeys,
                                     at<double>(ws, L.inv), L.Tp, scale, at<double>(ws, L.dvec), pg, dsg, L.Tp,
                                     L.Tp * L.Tp, s));
    hipLaunchKernelGGL(biased_dbias_kernel,
                       dim3(static_cast<unsigned>(ceil_div(static_cast<size_t>(L.n), 256)),
                            static_cast<unsigned>(L.n), static_cast<unsigned>(L.heads)),
                       dim3(256), 0, s, dsg, dbias, L.n, L.Tp);
    DLLM_TRY(check_launch("biased dbias"));
    // dq[t] = sum_j ds[t][j] k[j]; dk[j] = sum_t ds[t][j] q[t]; dv[j] = sum_t p[t][j] dout[t]
    DLLM_TRY(launch_attn_tiles(biased_sum(L, seg, dpt, k, L.hd, dq, nullptr), s));
    AttnTileCall kc = biased_sum(L, seg, dsg, q, L.hd, dk, nullptr);
    AttnTileCall vc = biased_sum(L, seg, pg, dout, L.vd, dv, nullptr);
    if (L.hd == L.vd) {
        kc.second = true;
        kc.A2 = vc.A;
        kc.B2 = vc.B;
        kc.C2 = vc.C;
        return launch_attn_tiles(kc, s);
    }
    DLLM_TRY(launch_attn_tiles(kc, s));
    return launch_attn_tiles(vc, s);
}

}  // namespace

}  // namespace dllm_hip

using namespace dllm_hip;

extern "C" {

int dllm_hip_gelu(const float* x, float* out, size_t n, void* stream) {
    if (n == 0) return kOk;
    DLLM_REQUIRE(x && out, "null argument");
    hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(static_cast<int64_t>(n), 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, out, static_cast<int64_t>(n));
    return check_launch("gelu");
}

int dllm_hip_gelu_backward(const float* x, const float* dy, float* out, size_t n, void* stream) {
    if (n == 0) return kOk;
    DLLM_REQUIRE(x && dy && out, "null argument");
    hipLaunchKernelGGL(gelu_backward_kernel, dim3(blocks_for(static_cast<int64_t>(n), 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, dy, out, static_cast<int64_t>(n));
    return check_launch("gelu_backward");
}

int dllm_hip_layer_norm(const float* x, const float* w, const float* b, float* out, size_t rows, size_t dim,
                        double eps, void* stream) {
    if (rows == 0 || dim == 0) return kOk;
    DLLM_REQUIRE(x && w && b && out, "null argument");
    hipLaunchKernelGGL(layer_norm_kernel, dim3(blocks_for(static_cast<int64_t>(rows), kLnRows)), dim3(64), 0,
                       static_cast<hipStream_t>(stream), x, w, b, out, static_cast<int64_t>(rows),
                       static_cast<int64_t>(dim), eps);
    return check_launch("layer_norm");
}

size_t dllm_hip_layer_norm_backward_workspace(size_t rows) { return round_up(rows * 2 * sizeof(double), 256); }

int dllm_hip_layer_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                                 size_t rows, size_t dim, double eps, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_layer_norm_backward_workspace(rows),
                 "workspace too small for layer_norm_backward");
    if (dim == 0) return kOk;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (rows == 0) {  // no rows: the column sums are +0.0
        if (dw) DLLM_TRY(check_hip(hipMemsetAsync(dw, 0, dim * sizeof(float), s), "memset"));
        if (db) DLLM_TRY(check_hip(hipMemsetAsync(db, 0, dim * sizeof(float), s), "memset"));
        return kOk;
    }
    DLLM_REQUIRE(x && w && dy && workspace, "null argument");
    double* stats = static_cast<double*>(workspace);
    hipLaunchKernelGGL(layer_norm_backward_rows_kernel, dim3(blocks_for(static_cast<int64_t>(rows), kLnRows)),
                       dim3(64), 0, s, x, w, dy, dx, stats, static_cast<int64_t>(rows), static_cast<int64_t>(dim), eps);
    DLLM_TRY(check_launch("layer_norm_backward rows"));
    if (!dw && !db) return kOk;
    const bool aligned = dim % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(dy) % 16 == 0;
    hipLaunchKernelGGL(aligned ? layer_norm_backward_cols_lds_kernel : layer_norm_backward_cols_kernel,
                       dim3(blocks_for(static_cast<int64_t>(dim), kLnColWidth)), dim3(1024), 0, s, x, dy, stats, dw,
                       db, static_cast<int64_t>(rows), static_cast<int64_t>(dim));
    return check_launch("layer_norm_backward columns");
}

size_t dllm_hip_biased_attention_workspace(size_t q_len, size_t kv_len, size_t heads, size_t head_dim,
                                           size_t value_dim) {
    if (biased_fast(q_len, kv_len, heads, head_dim, value_dim))
        return biased_layout(q_len, heads, head_dim, value_dim).forward;
    return round_up(q_len * heads * kv_len * sizeof(double), 256);
}

int dllm_hip_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out,
                              size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                              double scale, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_biased_attention_workspace(q_len, kv_len, heads, head_dim, value_dim),
                 "workspace too small for biased_attention");
    if (q_len == 0 || heads == 0) return kOk;
    DLLM_REQUIRE(q && out && (kv_len == 0 || (k && v && bias && workspace)), "null argument");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (biased_fast(q_len, kv_len, heads, head_dim, value_dim))
        return biased_forward_fast(q, k, v, bias, out, biased_layout(q_len, heads, head_dim, value_dim), scale,
                                   workspace, st);
    const BiasedShape s{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(heads),
                        static_cast<int64_t>(head_dim), static_cast<int64_t>(value_dim), scale};
    hipLaunchKernelGGL(biased_attention_kernel, dim3(static_cast<unsigned>(q_len * heads)), dim3(64), 0, st, q, k, v,
                       bias, out, static_cast<double*>(workspace), s);
    return check_launch("biased_attention");
}

int dllm_hip_biased_attention_weights(const float* q, const float* k, const float* bias, float* out, size_t q_len,
                                      size_t kv_len, size_t heads, size_t head_dim, double scale, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    // the forward's workspace with value_dim = 4 (the value sums are not formed)
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_biased_attention_workspace(q_len, kv_len, heads, head_dim, 4),
                 "workspace too small for biased_attention_weights");
    if (q_len == 0 || heads == 0 || kv_len == 0) return kOk;
    DLLM_REQUIRE(q && k && bias && out && workspace, "null argument");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (biased_fast(q_len, kv_len, heads, head_dim, 4)) {
        const BiasedLayout L = biased_layout(q_len, heads, head_dim, 4);
        DLLM_TRY(biased_probabilities_fast(q, k, bias, L, scale, workspace, st));
        const unsigned tiles = static_cast<unsigned>(ceil_div(q_len, 64));
        hipLaunchKernelGGL(biased_weights_kernel, dim3(tiles, tiles, static_cast<unsigned>(heads)), dim3(256), 0, st,
                           at<double>(workspace, L.et), at<double>(workspace, L.inv), out, L.n, L.Tp, L.heads);
        return check_launch("biased_attention_weights");
    }
    const BiasedShape s{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(heads),
                        static_cast<int64_t>(head_dim), 0, scale};
    hipLaunchKernelGGL(biased_weights_rows_kernel, dim3(static_cast<unsigned>(q_len * heads)), dim3(64), 0, st, q, k,
                       bias, out, static_cast<double*>(workspace), s);
    return check_launch("biased_attention_weights");
}

size_t dllm_hip_biased_attention_backward_workspace(size_t q_len, size_t kv_len, size_t heads, size_t head_dim,
                                                    size_t value_dim) {
    if (biased_fast(q_len, kv_len, heads, head_dim, value_dim))
        return biased_layout(q_len, heads, head_dim, value_dim).backward;
    return 2 * round_up(q_len * heads * kv_len * sizeof(double), 256);
}

int dllm_hip_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                       const float* dout, float* dq, float* dk, float* dv, float* dbias,
                                       size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                                       double scale, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >=
                     dllm_hip_biased_attention_backward_workspace(q_len, kv_len, heads, head_dim, value_dim),
                 "workspace too small for biased_attention_backward");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (biased_fast(q_len, kv_len, heads, head_dim, value_dim)) {
        DLLM_REQUIRE(q && k && v && bias && dout && dq && dk && dv && dbias && workspace, "null argument");
        return biased_backward_fast(q, k, v, bias, dout, dq, dk, dv, dbias,
                                    biased_layout(q_len, heads, head_dim, value_dim), scale, workspace, st);
    }
    const BiasedShape s{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(heads),
                        static_cast<int64_t>(head_dim), static_cast<int64_t>(value_dim), scale};
    double* p_save = static_cast<double*>(workspace);
    double* ds_save = reinterpret_cast<double*>(static_cast<char*>(workspace) +
                                                round_up(q_len * heads * kv_len * sizeof(double), 256));
    if (q_len > 0 && heads > 0) {
        DLLM_REQUIRE(q && dout && dq && (kv_len == 0 || (k && v && bias && dbias && workspace)), "null argument");
        hipLaunchKernelGGL(biased_attention_backward_rows_kernel, dim3(static_cast<unsigned>(q_len * heads)), dim3(64),
                           0, st, q, k, v, bias, dout, dq, dbias, p_save, ds_save, s);
        DLLM_TRY(check_launch("biased_attention_backward rows"));
    }
    const int64_t n = static_cast<int64_t>(kv_len * heads * (head_dim + value_dim));
    if (n == 0) return kOk;
    DLLM_REQUIRE(dk && dv, "null argument");
    hipLaunchKernelGGL(biased_attention_backward_kv_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, q, dout,
                       p_save, ds_save, dk, dv, s);
    return check_launch("biased_attention_backward keys");
}

}  // extern "C"
