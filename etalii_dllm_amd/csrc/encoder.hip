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

unsigned blocks_for(int64_t n, int per) { return static_cast<unsigned>(ceil_div(static_cast<size_t>(n), per)); }

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

size_t dllm_hip_biased_attention_workspace(size_t q_len, size_t kv_len, size_t heads) {
    return round_up(q_len * heads * kv_len * sizeof(double), 256);
}

int dllm_hip_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out,
                              size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                              double scale, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_biased_attention_workspace(q_len, kv_len, heads),
                 "workspace too small for biased_attention");
    if (q_len == 0 || heads == 0) return kOk;
    DLLM_REQUIRE(q && out && (kv_len == 0 || (k && v && bias && workspace)), "null argument");
    const BiasedShape s{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(heads),
                        static_cast<int64_t>(head_dim), static_cast<int64_t>(value_dim), scale};
    hipLaunchKernelGGL(biased_attention_kernel, dim3(static_cast<unsigned>(q_len * heads)), dim3(64), 0,
                       static_cast<hipStream_t>(stream), q, k, v, bias, out, static_cast<double*>(workspace), s);
    return check_launch("biased_attention");
}

size_t dllm_hip_biased_attention_backward_workspace(size_t q_len, size_t kv_len, size_t heads) {
    return 2 * dllm_hip_biased_attention_workspace(q_len, kv_len, heads);
}

int dllm_hip_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                       const float* dout, float* dq, float* dk, float* dv, float* dbias,
                                       size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                                       double scale, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_biased_attention_backward_workspace(q_len, kv_len, heads),
                 "workspace too small for biased_attention_backward");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const BiasedShape s{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(heads),
                        static_cast<int64_t>(head_dim), static_cast<int64_t>(value_dim), scale};
    double* p_save = static_cast<double*>(workspace);
    double* ds_save = reinterpret_cast<double*>(static_cast<char*>(workspace) +
                                                dllm_hip_biased_attention_workspace(q_len, kv_len, heads));
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
