// Row-local and elementwise kernels of the step: RMSNorm forward and backward, the column sums behind the norm weight
// and bias gradients, RoPE, SiLU/SwiGLU and their gradients, and the float32 glue between them.
//
// Reductions that the reference runs as one serial double chain per row (sum of squares, the backward dot) are run
// by lane 0 of the row's wave, in index order, after the other lanes are done loading; the per-element work around
// them is spread over the 64 lanes. Every float32 glue operation is one IEEE float op per element, in the
// reference's operand order.
#include <initializer_list>

#include <algorithm>

#include "common.h"
#include "devmath.h"
#include "kernels.h"
#include "lds_copy.h"

namespace dllm_hip {

namespace {

// The forward scale (nn.hpp:401-404): w, or 1 + w with the unit offset.
__device__ __forceinline__ double norm_scale(const float* w, int64_t i, int unit_offset) {
    if (w == nullptr) return 1.0;
    return unit_offset ? 1.0 + static_cast<double>(w[i]) : static_cast<double>(w[i]);
}

// The backward scale (grad.hpp:81,93): offset + w with offset 0 or 1 (so a -0.0 weight reads as +0.0, as there).
__device__ __forceinline__ double norm_scale_backward(const float* w, int64_t i, int unit_offset) {
    if (w == nullptr) return 1.0;
    return (unit_offset ? 1.0 : 0.0) + static_cast<double>(w[i]);
}

constexpr int kNormRows = 4;  // rows per 256-thread workgroup of the norm kernels (one per wave)

// Adds terms[0 .. n) to `chain` in index order, reading them from LDS 16 at a time ahead of the dependent adds.
__device__ __forceinline__ void chain_add(double& chain, const double* terms, int n) {
    int k = 0;
    for (; k + 16 <= n; k += 16) {
        double v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = terms[k + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) chain += v[u];
    }
    for (; k < n; ++k) chain += terms[k];
}

// rms_norm (nn.hpp:391-408) and rms_norm_backward's dx (grad.hpp:83-104), kNormRows rows per workgroup. Per row the serial
// chains run one lane per row out of LDS: the four waves stage the terms of kNormRows rows x 64 columns (x^2, and for
// the backward (g dy) x) in one of two buffers, then lanes 0 .. kNormRows - 1 of wave 0 add the squares and the next
// kNormRows lanes the products
// in ascending column order, while the next 64 columns' loads are in flight. Then every thread writes its elements:
//   forward   out = f32((x inv) scale),              inv = 1 / sqrt(sum x^2 / dim + eps)
//   backward  dx = f32((inv g) dy - x coef) (+ addend), coef = D inv inv inv / dim, D = sum (g dy) x
template <bool kBackward>
__global__ __launch_bounds__(256) void norm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ dy, float* __restrict__ out,
                                                        const float* __restrict__ addend, int64_t rows, int64_t dim,
                                                        double eps, int unit_offset, double* __restrict__ inv_out) {
    constexpr int kPer = kNormRows / 4;  // rows each wave stages
    __shared__ double squares[2][kNormRows][65];
    __shared__ double products[kBackward ? 2 : 1][kBackward ? kNormRows : 1][65];
    __shared__ double row_inv[kNormRows], row_coef[kNormRows];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kNormRows;
    const int64_t nrows = rows - r0 < kNormRows ? rows - r0 : kNormRows;
    const int64_t chunks = (dim + 63) / 64;
    float xv[kPer], dv[kPer];
    auto load = [&](int64_t c) {  // this thread's x (and dy) of chunk c, rows wave * kPer + k
        const int64_t col = c * 64 + lane;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int r = wave * kPer + k;
            const bool in = col < dim && r < nrows;
            xv[k] = in ? x[(r0 + r) * dim + col] : 0.0f;
            if (kBackward) dv[k] = in ? dy[(r0 + r) * dim + col] : 0.0f;
        }
    };
    auto store = [&](int64_t c) {
        const int64_t col = c * 64 + lane;
        const double g = kBackward && col < dim ? norm_scale_backward(w, col, unit_offset) : 0.0;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int r = wave * kPer + k;
            const double xd = static_cast<double>(xv[k]);
            squares[c & 1][r][lane] = xd * xd;
            if (kBackward) products[c & 1][r][lane] = g * static_cast<double>(dv[k]) * xd;
        }
    };
    double chain = 0.0;  // wave 0: lane r < kNormRows the squares of row r, lane kNormRows + r the products of row r
    load(0);
    store(0);
    __syncthreads();
    for (int64_t c = 0; c < chunks; ++c) {
        if (c + 1 < chunks) load(c + 1);
        const int n = static_cast<int>(dim - c * 64 < 64 ? dim - c * 64 : 64);
        if (wave == 0) {
            if (lane < kNormRows)
                chain_add(chain, &squares[c & 1][lane][0], n);
            else if (kBackward && lane < 2 * kNormRows)
                chain_add(chain, &products[c & 1][lane - kNormRows][0], n);
        }
        if (c + 1 < chunks) store(c + 1);
        __syncthreads();
    }
    if (wave == 0 && lane < kNormRows && lane < nrows) {
        const double inv = 1.0 / sqrt(chain / static_cast<double>(dim) + eps);
        row_inv[lane] = inv;
        if (inv_out) inv_out[r0 + lane] = inv;
    }
    __syncthreads();
    if (kBackward && wave == 0 && lane >= kNormRows && lane < 2 * kNormRows && lane - kNormRows < nrows) {
        const double inv = row_inv[lane - kNormRows];
        row_coef[lane - kNormRows] = chain * inv * inv * inv / static_cast<double>(dim);
    }
    __syncthreads();
    for (int r = wave; r < nrows; r += 4) {
        const double inv = row_inv[r];
        const int64_t base = (r0 + r) * dim;
        if (kBackward) {
            const double coef = row_coef[r];
#pragma unroll 8
            for (int64_t i = lane; i < dim; i += 64) {
                const double g = norm_scale_backward(w, i, unit_offset);
                float v = static_cast<float>(inv * g * static_cast<double>(dy[base + i]) -
                                             static_cast<double>(x[base + i]) * coef);
                if (addend) v = addend[base + i] + v;
                out[base + i] = v;
            }
        } else {
#pragma unroll 8
            for (int64_t i = lane; i < dim; i += 64)
                out[base + i] = static_cast<float>(static_cast<double>(x[base + i]) * inv * norm_scale(w, i, unit_offset));
        }
    }
}

// part[s][i] = f32(sum over rows of segment s ascending of term(r, i)): kind 0 term = dy (db, grad.hpp:52-54),
// kind 1 term = (dy x) inv_rms[r] (norm weight, grad.hpp:95).
constexpr int kColSegs = 64;  // segments per column-sums launch

struct ColSegments {
    int64_t off[kColSegs + 1];
};

// part[s][i] = f32(sum over rows r of segment s, ascending, of term(r, i)) for 64 columns per workgroup: the four
// waves stage the terms of 64 rows x 64 columns in one of two LDS buffers, then one wave runs the 64 serial
// additions per column while the next 64 rows' loads are in flight.
__global__ __launch_bounds__(256) void column_partial_kernel(int kind, const float* __restrict__ dy,
                                                             const float* __restrict__ x,
                                                             const double* __restrict__ inv, int64_t dim,
                                                             ColSegments seg, float* __restrict__ part) {
    __shared__ double terms[2][64][64];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 64 + lane;
    const int64_t col = i < dim ? i : dim - 1;
    const int64_t r0 = seg.off[blockIdx.y], r1 = seg.off[blockIdx.y + 1];
    const int64_t blocks = (r1 - r0 + 63) / 64;
    double tv[16];
    auto load = [&](int64_t b) {  // rows wave + 4 k of block b
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int64_t r = r0 + b * 64 + wave + 4 * k;
            double t = 0.0;
            if (r < r1) {
                t = static_cast<double>(dy[r * dim + col]);
                if (kind != 0) t = t * static_cast<double>(x[r * dim + col]) * inv[r];
            }
            tv[k] = t;
        }
    };
    auto store = [&](int64_t b) {
#pragma unroll
        for (int k = 0; k < 16; ++k) terms[b & 1][wave + 4 * k][lane] = tv[k];
    };
    double acc = 0.0;
    if (blocks > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int64_t b = 0; b < blocks; ++b) {
        if (b + 1 < blocks) load(b + 1);
        const int n = static_cast<int>(r1 - r0 - b * 64 < 64 ? r1 - r0 - b * 64 : 64);
        if (wave == 0) {
            int row = 0;
            for (; row + 16 <= n; row += 16) {
                double v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = terms[b & 1][row + u][lane];
#pragma unroll
                for (int u = 0; u < 16; ++u) acc += v[u];
            }
            for (; row < n; ++row) acc += terms[b & 1][row][lane];
        }
        if (b + 1 < blocks) store(b + 1);
        __syncthreads();
    }
    if (wave == 0 && i < dim) part[static_cast<int64_t>(blockIdx.y) * dim + i] = static_cast<float>(acc);
}

// The same sums with the raw rows copied straight to LDS (global_load_lds) kCsRing chunks of 64 rows ahead, tracked by
// explicit counter waits (dim % 4 == 0, 16-byte aligned dy and x). A 1024-thread workgroup takes 16 columns of one
// segment: waves 0-3 copy dy (16 rows each, 4 lanes per row), waves 4-7 x, waves 8 and 9 the rows' inv_rms as
// 4-byte halves (kind 1); one copy per wave per chunk. Thread t forms the term of row slot t / 16, column t % 16
// into LDS, and lanes 0-15 of wave 0 add the previous chunk's terms onto the column chains in row order. At
// 8192 x 896 (56 workgroups) the launch takes 85 us: 33 us without the chains, 42 us with the chains but no terms
// formed; a wave that only runs the chains (two chunks behind, three term buffers) measured no faster.
constexpr int kCsRing = 8;

template <int kC>
struct CsSlot {
    float dy[64][kC];
    float x[64][kC];
    double inv[64];
};

template <int kC>
__global__ __launch_bounds__(64 * kC) void column_partial_lds_kernel(int kind, const float* __restrict__ dy,
                                                                     const float* __restrict__ x,
                                                                     const double* __restrict__ inv, int64_t dim,
                                                                     ColSegments seg, float* __restrict__ part) {
    constexpr int kLanesPerRow = kC / 4;            // 16-byte pieces of a row's kC columns
    constexpr int kRowsPerCopy = 64 / kLanesPerRow;  // rows one wave's copy covers
    constexpr int kWaves = 64 / kRowsPerCopy;         // waves copying dy (and as many x)
    __shared__ __align__(16) CsSlot<kC> ring[kCsRing];
    __shared__ double terms[2][64][kC];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int c16 = tid % kC, slot = tid / kC;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kC;
    const int64_t r0 = seg.off[blockIdx.y], r1 = seg.off[blockIdx.y + 1];
    const int64_t chunks = (r1 - r0 + 63) / 64;
    double acc = 0.0;
    if (chunks > 0) {
        const auto issue = [&](int64_t c) {
            const int64_t cc = c < chunks ? c : chunks - 1;
            CsSlot<kC>& dst = ring[cc % kCsRing];
            const int64_t base = r0 + cc * 64;
            if (wave < 2 * kWaves) {
                if (wave >= kWaves && kind == 0) return;
                const int w = wave % kWaves;
                const int rr = kRowsPerCopy * w + lane / kLanesPerRow;
                const int64_t r = base + rr < r1 ? base + rr : r1 - 1;
                const int64_t g = col0 + 4 * (lane % kLanesPerRow) < dim ? col0 + 4 * (lane % kLanesPerRow) : dim - 4;
                copy16_to_lds((wave < kWaves ? dy : x) + r * dim + g,
                              wave < kWaves ? &dst.dy[kRowsPerCopy * w][0] : &dst.x[kRowsPerCopy * w][0]);
            } else if (wave < 2 * kWaves + 2 && kind != 0) {
                const int half = wave - 2 * kWaves;  // rows 32 half .. 32 half + 31, two 4-byte lanes each
                const int64_t rr = 32 * half + lane / 2;
                const int64_t r = base + rr < r1 ? base + rr : r1 - 1;
                copy4_to_lds(reinterpret_cast<const char*>(inv + r) + 4 * (lane & 1), &dst.inv[32 * half]);
            }
        };
        for (int k = 0; k < kCsRing - 1; ++k) issue(k);
        for (int64_t c = 0; c <= chunks; ++c) {
            // chunk c landed (kCsRing - 2 newer copies may be pending per wave), the previous terms are written, and
            // every wave is done reading the ring slot the next copy refills
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kCsRing - 2) : "memory");
            issue(c + kCsRing - 1);
            const CsSlot<kC>& src = ring[(c < chunks ? c : chunks - 1) % kCsRing];
            const int buf = static_cast<int>(c & 1);
            double t = static_cast<double>(src.dy[slot][c16]);
            if (kind != 0) t = t * static_cast<double>(src.x[slot][c16]) * src.inv[slot];
            terms[buf][slot][c16] = t;
            if (c > 0 && tid < kC) {
                const double(&tp)[64][kC] = terms[buf ^ 1];
                const int64_t rs = (c - 1) * 64;
                const int n = r1 - r0 - rs < 64 ? static_cast<int>(r1 - r0 - rs) : 64;
                if (n == 64) {
                    // 16 rows' terms read ahead of the 16 adds they feed, the next 16 issued before those adds: the
                    // scheduling barriers keep the compiler from moving the reads down next to their adds, which
                    // left one read in flight and an LDS latency per two adds
                    double cur[16], nxt[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) cur[u] = tp[u][tid];
#pragma unroll
                    for (int blk = 0; blk < 4; ++blk) {
                        if (blk < 3) {
#pragma unroll
                            for (int u = 0; u < 16; ++u) nxt[u] = tp[16 * (blk + 1) + u][tid];
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int u = 0; u < 16; ++u) acc += cur[u];
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int u = 0; u < 16; ++u) cur[u] = nxt[u];
                    }
                } else {
                    for (int rr = 0; rr < n; ++rr) acc += tp[rr][tid];
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the end drain before exit
    }
    if (tid < kC && col0 + tid < dim)
        part[static_cast<int64_t>(blockIdx.y) * dim + col0 + tid] = static_cast<float>(acc);
}

// out[i] = part[0][i] + part[1][i] + ... in float, segment order (trainer.py:328-332: the first copied).
// out = part[0] + part[1] + ... in float, window order, the first copied; with factors, each window's part is first
// multiplied by its factor (window s adds f32(part[s] * w[s])).
__global__ __launch_bounds__(256) void segment_float_sum_kernel(const float* __restrict__ part, int64_t dim, int nseg,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ colscale,
                                                                float* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= dim) return;
    // each window's column sum times its column factor (when given), then its window factor, added in window order
    const auto term = [&](int s) {
        float v = part[static_cast<int64_t>(s) * dim + i];
        if (colscale) v = v * colscale[i];
        if (w) v = v * w[s];
        return v;
    };
    float t = term(0);
    for (int s = 1; s < nseg; ++s) t = t + term(s);
    out[i] = t;
}

// cos and sin of positions[t] * inv_freq[i] with the portable sin/cos (nn.hpp:508-513).
__global__ __launch_bounds__(256) void rope_table_kernel(const int64_t* __restrict__ positions, int64_t n,
                                                         const double* __restrict__ inv_freq, int64_t half,
                                                         double* __restrict__ ct, double* __restrict__ st) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= n * half) return;
    const int64_t t = idx / half, i = idx % half;
    double c, sn;
    dsincos(positions ? static_cast<double>(positions[t]) : static_cast<double>(t), inv_freq[i], &sn, &c);
    ct[idx] = c;
    st[idx] = sn;
}

// rope (nn.hpp:515-527); inverse negates the sine exactly.
// Element k of row (token t, head h) of one tensor's rotation: pair k, or a pass-through value past rotary_dim.
__device__ __forceinline__ void rope_element(int64_t t, int64_t h, int64_t k, const float* __restrict__ x,
                                             const int64_t* __restrict__ pos_index, const double* __restrict__ ct,
                                             const double* __restrict__ st, float* __restrict__ out, int64_t heads,
                                             int64_t head_dim, int64_t rotary_dim, int interleaved, int inverse) {
    const int64_t half = rotary_dim / 2;
    const float* xh = x + (t * heads + h) * head_dim;
    float* oh = out + (t * heads + h) * head_dim;
    if (k >= half) {
        const int64_t i = rotary_dim + (k - half);
        oh[i] = xh[i];
        return;
    }
    const int64_t row = pos_index ? pos_index[t] : t;
    const double c = ct[row * half + k];
    const double s = inverse ? -st[row * half + k] : st[row * half + k];
    const int64_t i0 = interleaved ? 2 * k : k;
    const int64_t i1 = interleaved ? 2 * k + 1 : k + half;
    const double a = xh[i0];
    const double b = xh[i1];
    oh[i0] = static_cast<float>(a * c - b * s);
    oh[i1] = static_cast<float>(a * s + b * c);
}

// How a wave's lanes cover rows of per_head elements: one row at a time (lane k takes k, k + 64, ...), or, for rows of
// at most 32 elements dividing 64, 64 / per_head rows at once (lane = sub row x per_head + k).
struct RopeLanes {
    int64_t rows, sub, k0, step;
};

__device__ __forceinline__ RopeLanes rope_lanes(int64_t per_head) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    if (per_head <= 32 && 64 % per_head == 0) return RopeLanes{64 / per_head, lane / per_head, lane % per_head, per_head};
    return RopeLanes{1, 0, lane, 64};
}

// row / heads: a 32-bit division (a few instructions) when every row index fits 32 bits, as it does for any tensor
// below 2^32 rows; the 64-bit one is a long software sequence, paid per lane when a wave covers several rows.
__device__ __forceinline__ int64_t row_token(int64_t row, int64_t heads, int64_t rows) {
    if (rows <= 0xffffffffLL) return static_cast<uint32_t>(row) / static_cast<uint32_t>(heads);
    return row / heads;
}

__global__ __launch_bounds__(256) void rope_kernel(const float* __restrict__ x, const int64_t* __restrict__ pos_index,
                                                   const double* __restrict__ ct, const double* __restrict__ st,
                                                   float* __restrict__ out, int64_t tokens, int64_t heads,
                                                   int64_t head_dim, int64_t rotary_dim, int interleaved, int inverse) {
    // one wave per (token, head) row at a time, or several rows per wave for short rows, as rope_pair_kernel below
    const int64_t per_head = rotary_dim / 2 + head_dim - rotary_dim;
    const RopeLanes rl = rope_lanes(per_head);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * rl.rows + rl.sub;
         row - rl.sub < tokens * heads; row += waves * rl.rows) {
        if (row >= tokens * heads) continue;
        const int64_t t = row_token(row, heads, tokens * heads), h = row - t * heads;
        for (int64_t k = rl.k0; k < per_head; k += rl.step)
            rope_element(t, h, k, x, pos_index, ct, st, out, heads, head_dim, rotary_dim, interleaved, inverse);
    }
}

// rope with the cos/sin computed in place (rows of at most 64 elements): one wave per token at a time; lane
// (sub, k) = (lane / per_head, lane % per_head) computes the cos and sin of pair k once, exactly as rope_table_kernel
// does, and rotates pair k of heads sub, sub + G, ... (G = 64 / per_head rows per wave), four heads' loads in flight
// at a time. No table is written or read, and one launch replaces two. (Splitting a token's heads over more waves,
// and issuing the first loads before the cos and sin, both measured slower at 8192 tokens x 14 heads of 64.)
__global__ __launch_bounds__(256) void rope_direct_kernel(const float* __restrict__ x,
                                                          const int64_t* __restrict__ positions,
                                                          const double* __restrict__ inv_freq,
                                                          float* __restrict__ out, int64_t tokens, int64_t heads,
                                                          int64_t head_dim, int64_t rotary_dim, int interleaved,
                                                          int inverse) {
    const int64_t half = rotary_dim / 2, per_head = half + head_dim - rotary_dim;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int g = static_cast<int>(64 / per_head);
    const int sub = lane / static_cast<int>(per_head), k = lane - sub * static_cast<int>(per_head);
    if (sub >= g) return;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); t < tokens; t += waves) {
        const float* xt = x + t * heads * head_dim;
        float* ot = out + t * heads * head_dim;
        if (k >= half) {
            const int64_t i = rotary_dim + (k - half);
            for (int64_t h = sub; h < heads; h += g) ot[h * head_dim + i] = xt[h * head_dim + i];
            continue;
        }
        double c, sn;
        dsincos(positions ? static_cast<double>(positions[t]) : static_cast<double>(t), inv_freq[k], &sn, &c);
        const double sv = inverse ? -sn : sn;
        const int64_t i0 = interleaved ? 2 * k : k;
        const int64_t i1 = interleaved ? 2 * k + 1 : k + half;
        int64_t h = sub;
        for (; h + 3 * g < heads; h += 4 * g) {
            double a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u] = xt[(h + u * g) * head_dim + i0];
                b[u] = xt[(h + u * g) * head_dim + i1];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ot[(h + u * g) * head_dim + i0] = static_cast<float>(a[u] * c - b[u] * sv);
                ot[(h + u * g) * head_dim + i1] = static_cast<float>(a[u] * sv + b[u] * c);
            }
        }
        for (; h < heads; h += g) {
            const double a = xt[h * head_dim + i0], b = xt[h * head_dim + i1];
            ot[h * head_dim + i0] = static_cast<float>(a * c - b * sv);
            ot[h * head_dim + i1] = static_cast<float>(a * sv + b * c);
        }
    }
}

// Two tensors of the same tokens (the queries and the keys) in one launch, one wave per (token, head) row at a time,
// or 64 / per_head rows at once for rows of at most 32 elements (rope_lanes): lane k takes pairs k, k + 64, ... of its
// row (coalesced loads and stores), its token a 32-bit division (row_token). Rows [0, tokens heads1) are the first
// tensor's, the next tokens heads2 the second's. (One thread per pair with 64-bit index divisions made the kernel
// compute-bound: 3.3 TB/s at c3's 8192 x 1792 values.)
__global__ __launch_bounds__(256) void rope_pair_kernel(const float* __restrict__ x1, float* __restrict__ out1,
                                                        int64_t heads1, const float* __restrict__ x2,
                                                        float* __restrict__ out2, int64_t heads2,
                                                        const int64_t* __restrict__ pos_index,
                                                        const double* __restrict__ ct, const double* __restrict__ st,
                                                        int64_t tokens, int64_t head_dim, int64_t rotary_dim,
                                                        int inverse) {
    const int64_t per_head = rotary_dim / 2 + (head_dim - rotary_dim);
    const int64_t rows1 = tokens * heads1, rows = rows1 + tokens * heads2;
    const RopeLanes rl = rope_lanes(per_head);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * rl.rows + rl.sub;
         row - rl.sub < rows; row += waves * rl.rows) {
        if (row >= rows) continue;
        const bool second = row >= rows1;
        const int64_t r = second ? row - rows1 : row;
        const int64_t heads = second ? heads2 : heads1;
        const int64_t t = row_token(r, heads, rows), h = r - t * heads;
        for (int64_t k = rl.k0; k < per_head; k += rl.step)
            rope_element(t, h, k, second ? x2 : x1, pos_index, ct, st, second ? out2 : out1, heads, head_dim,
                         rotary_dim, 0, inverse);
    }
}

__global__ __launch_bounds__(256) void silu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = dsilu(x[i]);
}

// gelu_tanh (nn.hpp:481-485): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), in double, rounded once.
__device__ __forceinline__ float dgelu_tanh(float x) {
    const double c = 7.97884560802865355879e-01;  // sqrt(2 / pi)
    const double d = x;
    return static_cast<float>(0.5 * d * (1.0 + dtanh(c * (d + 0.044715 * d * d * d))));
}

__global__ __launch_bounds__(256) void gelu_tanh_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                        int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = dgelu_tanh(x[i]);
}

// The gated GELU-tanh activation (gated_activation<gelu_tanh>, nn.hpp:488-492): the activation rounded, then a float
// multiply.
__global__ __launch_bounds__(256) void geglu_tanh_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                         float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = dgelu_tanh(gate[i]) * up[i];
}

// gelu_tanh_backward (grad.hpp:183-191): dy times 0.5 (1 + t) + 0.5 x (1 - t^2) sqrt(2/pi) (1 + 3 0.044715 x^2),
// t = tanh(sqrt(2/pi) (x + 0.044715 x^3)), in double, rounded once.
__device__ __forceinline__ float dgelu_tanh_backward(float x, float dy) {
    const double c = 7.97884560802865355879e-01;  // sqrt(2 / pi)
    const double d = x;
    const double t = dtanh(c * (d + 0.044715 * d * d * d));
    const double slope = 0.5 * (1.0 + t) + 0.5 * d * (1.0 - t * t) * c * (1.0 + 3.0 * 0.044715 * d * d);
    return static_cast<float>(static_cast<double>(dy) * slope);
}

// The gated MLP's activation: kAct 0 SiLU, 1 GELU with the tanh approximation (backprop.py:163-171).
template <int kAct>
__device__ __forceinline__ float gate_activation(float x) {
    return kAct == 1 ? dgelu_tanh(x) : dsilu(x);
}
template <int kAct>
__device__ __forceinline__ float gate_activation_backward(float x, float dy) {
    return kAct == 1 ? dgelu_tanh_backward(x, dy) : dsilu_backward(x, dy);
}

template <int kAct>
__global__ __launch_bounds__(256) void swiglu_forward_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                             float* __restrict__ gate_act, float* __restrict__ product,
                                                             int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float a = gate_activation<kAct>(gate[i]);
        if (gate_act) gate_act[i] = a;
        product[i] = a * up[i];
    }
}

// The same two kernels on 16-byte vectors (four independent elements per thread in flight), for 16-byte aligned
// arrays; the launchers run the scalar kernels on the last n % 4 elements.
__device__ __forceinline__ float4 load4(const float* p, int64_t q) { return reinterpret_cast<const float4*>(p)[q]; }
__device__ __forceinline__ void store4(float* p, int64_t q, float4 v) { reinterpret_cast<float4*>(p)[q] = v; }

__global__ __launch_bounds__(256) void swiglu_forward4_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                              float* __restrict__ gate_act, float* __restrict__ product,
                                                              int64_t n4) {
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < n4;
         q += static_cast<int64_t>(gridDim.x) * 256) {
        const float4 g = load4(gate, q), u = load4(up, q);
        const float4 a = {dsilu(g.x), dsilu(g.y), dsilu(g.z), dsilu(g.w)};
        if (gate_act) store4(gate_act, q, a);
        store4(product, q, float4{a.x * u.x, a.y * u.y, a.z * u.z, a.w * u.w});
    }
}

__global__ __launch_bounds__(256) void swiglu_backward4_kernel(const float* __restrict__ gate,
                                                               const float* __restrict__ up,
                                                               const float* __restrict__ gate_act,
                                                               const float* __restrict__ dproduct,
                                                               float* __restrict__ dgate, float* __restrict__ dup,
                                                               int64_t n4) {
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < n4;
         q += static_cast<int64_t>(gridDim.x) * 256) {
        const float4 dp = load4(dproduct, q), u = load4(up, q), g = load4(gate, q), a = load4(gate_act, q);
        store4(dgate, q, float4{dsilu_backward(g.x, dp.x * u.x), dsilu_backward(g.y, dp.y * u.y),
                                dsilu_backward(g.z, dp.z * u.z), dsilu_backward(g.w, dp.w * u.w)});
        store4(dup, q, float4{dp.x * a.x, dp.y * a.y, dp.z * a.z, dp.w * a.w});
    }
}

__global__ __launch_bounds__(256) void silu_backward_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                            float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = dsilu_backward(x[i], dy[i]);
}

// gelu_tanh_backward (grad.hpp:183-191) and softcap_backward (grad.hpp:193-197), elementwise, in double, rounded once.
__global__ __launch_bounds__(256) void gelu_tanh_backward_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ dy, float* __restrict__ out,
                                                                 int64_t n) {
    const double c = 7.97884560802865355879e-01;  // sqrt(2 / pi)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        (void)c;
        out[i] = dgelu_tanh_backward(x[i], dy[i]);
    }
}

__global__ __launch_bounds__(256) void softcap_backward_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                               float* __restrict__ out, int64_t n, double cap) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const double t = dtanh(static_cast<double>(x[i]) / cap);
        out[i] = static_cast<float>(static_cast<double>(dy[i]) * (1.0 - t * t));
    }
}

template <int kAct>
__global__ __launch_bounds__(256) void swiglu_backward_kernel(const float* __restrict__ gate,
                                                              const float* __restrict__ up,
                                                              const float* __restrict__ gate_act,
                                                              const float* __restrict__ dproduct,
                                                              float* __restrict__ dgate, float* __restrict__ dup,
                                                              int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float dp = dproduct[i];
        dgate[i] = gate_activation_backward<kAct>(gate[i], dp * up[i]);
        dup[i] = dp * gate_act[i];
    }
}

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ table,
                                                          const int64_t* __restrict__ index, float* __restrict__ out,
                                                          int64_t rows, int64_t dim) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    const float* src = table + index[r] * dim;
    for (int64_t i = threadIdx.x; i < dim; i += 256) out[r * dim + i] = src[i];
}

// Every non-null pointer 16-byte aligned.
bool aligned16(std::initializer_list<const float*> ptrs) {
    for (const float* p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}

unsigned elementwise_grid(int64_t n) {
    const int64_t blocks = (n + 255) / 256;
    return static_cast<unsigned>(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

int launch_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t dim, double eps, int unit_offset,
                    double* inv_rms, hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(dim > 0, "rms_norm needs a non-empty last dimension");
    hipLaunchKernelGGL(norm_rows_kernel<false>, dim3(static_cast<unsigned>(ceil_div(rows, kNormRows))), dim3(256), 0,
                       stream, x, w, nullptr, out, nullptr, rows, dim, eps, unit_offset, inv_rms);
    return check_launch("rms_norm");
}

int launch_rms_norm_backward_dx(const float* x, const float* w, const float* dy, float* dx, const float* addend,
                                int64_t rows, int64_t dim, double eps, int unit_offset, double* inv_rms,
                                hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(dim > 0, "rms_norm_backward needs a non-empty last dimension");
    hipLaunchKernelGGL(norm_rows_kernel<true>, dim3(static_cast<unsigned>(ceil_div(rows, kNormRows))), dim3(256), 0,
                       stream, x, w, dy, dx, addend, rows, dim, eps, unit_offset, inv_rms);
    return check_launch("rms_norm_backward");
}

int launch_segment_sums(const float* partial, int64_t dim, int nseg, const float* weights, float* out,
                        hipStream_t stream) {
    if (dim == 0) return kOk;
    hipLaunchKernelGGL(segment_float_sum_kernel, dim3(static_cast<unsigned>(ceil_div(dim, 256))), dim3(256), 0, stream,
                       partial, dim, nseg, weights, nullptr, out);
    return check_launch("segment sums");
}

int launch_column_sums(int kind, const float* dy, const float* x, const double* inv_rms, int64_t dim,
                       const int64_t* seg_host, int nseg, float* partial, float* out, hipStream_t stream,
                       const float* weights, const float* colscale) {
    if (dim == 0) return kOk;
    DLLM_REQUIRE(nseg >= 1, "column sums need a segment");
    DLLM_REQUIRE((nseg == 1 && !weights && !colscale) || partial != nullptr,
                 "column sums over several segments (or with factors) need a partial buffer");
    const bool direct = nseg == 1 && !weights && !colscale;
    const unsigned col_blocks = static_cast<unsigned>(ceil_div(dim, 64));
    // the direct-to-LDS kernel: whole 16-byte pieces of rows
    const bool ring = dim % 4 == 0 && reinterpret_cast<uintptr_t>(dy) % 16 == 0 &&
                      (kind == 0 || (reinterpret_cast<uintptr_t>(x) % 16 == 0 && inv_rms != nullptr));
    for (int s0 = 0; s0 < nseg; s0 += kColSegs) {
        const int count = nseg - s0 < kColSegs ? nseg - s0 : kColSegs;
        ColSegments seg{};
        for (int s = 0; s <= count; ++s) seg.off[s] = seg_host[s0 + s];
        float* part = direct ? out : partial + static_cast<int64_t>(s0) * dim;
        if (ring)
        {
            // 16, 8 or 4 columns per workgroup. For segments of 4096 rows or more, the narrowest that still puts
            // at most one workgroup on each CU: a narrower workgroup's smaller copies per chunk shorten its time
            // (one window of 8192 x 896: 84 us with 16 columns, 78 with 4), but workgroups sharing a CU slow each
            // other (8192 x 4864 with 4 columns, 1216 workgroups: 233 us against 155 with 16). Otherwise the fewest
            // rounds of workgroups over the CUs (their LDS rings hold 1, 3 or 6 per CU), the wider on a tie.
            const auto groups = [&](int c) { return ceil_div(dim, c) * count; };
            const auto rounds = [&](int c, int per_cu) {
                return ceil_div(groups(c), static_cast<int64_t>(per_cu) * 256);
            };
            int64_t longest = 0;
            for (int s = 0; s < count; ++s) longest = std::max<int64_t>(longest, seg.off[s + 1] - seg.off[s]);
            const int64_t r16 = rounds(16, 1), r8 = rounds(8, 3), r4 = rounds(4, 6);
            int kc = r16 <= r8 && r16 <= r4 ? 16 : r8 <= r4 ? 8 : 4;
            if (longest >= 4096 && groups(16) <= 256) kc = groups(4) <= 256 ? 4 : groups(8) <= 256 ? 8 : 16;
            if (kc == 16)
                hipLaunchKernelGGL(column_partial_lds_kernel<16>, dim3(static_cast<unsigned>(ceil_div(dim, 16)),
                                                                       static_cast<unsigned>(count)),
                                   dim3(1024), 0, stream, kind, dy, x, inv_rms, dim, seg, part);
            else if (kc == 8)
                hipLaunchKernelGGL(column_partial_lds_kernel<8>, dim3(static_cast<unsigned>(ceil_div(dim, 8)),
                                                                      static_cast<unsigned>(count)),
                                   dim3(512), 0, stream, kind, dy, x, inv_rms, dim, seg, part);
            else
                hipLaunchKernelGGL(column_partial_lds_kernel<4>, dim3(static_cast<unsigned>(ceil_div(dim, 4)),
                                                                      static_cast<unsigned>(count)),
                                   dim3(256), 0, stream, kind, dy, x, inv_rms, dim, seg, part);
        }
        else
            hipLaunchKernelGGL(column_partial_kernel, dim3(col_blocks, static_cast<unsigned>(count)), dim3(256), 0,
                               stream, kind, dy, x, inv_rms, dim, seg, part);
    }
    const unsigned blocks = static_cast<unsigned>(ceil_div(dim, 256));
    if (!direct)
        hipLaunchKernelGGL(segment_float_sum_kernel, dim3(blocks), dim3(256), 0, stream, partial, dim, nseg, weights,
                           colscale, out);
    return check_launch("column_sums");
}

int launch_rope_tables(const int64_t* positions, int64_t n, const double* inv_freq, int64_t half, double* cos_table,
                       double* sin_table, hipStream_t stream) {
    if (n * half == 0) return kOk;
    hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<unsigned>(ceil_div(n * half, 256))), dim3(256), 0, stream,
                       positions, n, inv_freq, half, cos_table, sin_table);
    return check_launch("rope_tables");
}

int launch_rope_pair(const float* x1, float* out1, int64_t heads1, const float* x2, float* out2, int64_t heads2,
                     const int64_t* pos_index, const double* cos_table, const double* sin_table, int64_t tokens,
                     int64_t head_dim, int64_t rotary_dim, int inverse, hipStream_t stream) {
    DLLM_REQUIRE(rotary_dim % 2 == 0 && rotary_dim <= head_dim, "rotary_dim must be even and at most head_dim");
    const int64_t n = tokens * (heads1 + heads2) * (rotary_dim / 2 + head_dim - rotary_dim);
    if (n == 0) return kOk;
    const int64_t rows = tokens * (heads1 + heads2);
    hipLaunchKernelGGL(rope_pair_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(rows, 4), 16384))),
                       dim3(256), 0, stream, x1, out1, heads1, x2, out2, heads2, pos_index, cos_table, sin_table,
                       tokens, head_dim, rotary_dim, inverse);
    return check_launch("rope");
}

int launch_rope(const float* x, const int64_t* pos_index, const double* cos_table, const double* sin_table,
                float* out, int64_t tokens, int64_t heads, int64_t head_dim, int64_t rotary_dim, int interleaved,
                int inverse, hipStream_t stream) {
    DLLM_REQUIRE(rotary_dim % 2 == 0 && rotary_dim <= head_dim, "rotary_dim must be even and at most head_dim");
    const int64_t n = tokens * heads * (rotary_dim / 2 + head_dim - rotary_dim);
    if (n == 0) return kOk;
    hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(tokens * heads, 4), 16384))),
                       dim3(256), 0, stream, x, pos_index, cos_table, sin_table, out, tokens, heads, head_dim,
                       rotary_dim, interleaved, inverse);
    return check_launch("rope");
}

int launch_rope_direct(const float* x, const int64_t* positions, const double* inv_freq, float* out, int64_t tokens,
                       int64_t heads, int64_t head_dim, int64_t rotary_dim, int interleaved, int inverse,
                       hipStream_t stream) {
    DLLM_REQUIRE(rotary_dim % 2 == 0 && rotary_dim <= head_dim, "rotary_dim must be even and at most head_dim");
    DLLM_REQUIRE(rotary_dim / 2 + head_dim - rotary_dim <= 64, "rope_direct: rows of at most 64 elements");
    if (tokens * heads * head_dim == 0) return kOk;
    hipLaunchKernelGGL(rope_direct_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(tokens, 4), 16384))),
                       dim3(256), 0, stream, x, positions, inv_freq, out, tokens, heads, head_dim, rotary_dim,
                       interleaved, inverse);
    return check_launch("rope");
}

int launch_silu(const float* x, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(silu_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, out, n);
    return check_launch("silu");
}

int launch_swiglu_forward(const float* gate, const float* up, float* gate_act, float* product, int64_t n,
                          hipStream_t stream, int activation) {
    if (n == 0) return kOk;
    if (activation == 1) {
        hipLaunchKernelGGL(swiglu_forward_kernel<1>, dim3(elementwise_grid(n)), dim3(256), 0, stream, gate, up,
                           gate_act, product, n);
        return check_launch("geglu");
    }
    const int64_t n4 = aligned16({gate, up, gate_act, product}) ? n / 4 : 0;
    if (n4 > 0)
        hipLaunchKernelGGL(swiglu_forward4_kernel, dim3(elementwise_grid(n4)), dim3(256), 0, stream, gate, up,
                           gate_act, product, n4);
    const int64_t d = 4 * n4;
    if (n > d)
        hipLaunchKernelGGL(swiglu_forward_kernel<0>, dim3(elementwise_grid(n - d)), dim3(256), 0, stream, gate + d,
                           up + d, gate_act ? gate_act + d : nullptr, product + d, n - d);
    return check_launch("swiglu");
}

// A plain device copy of n4 16-byte vectors, four in flight per thread, then the n % 16 tail bytes one by one.
__global__ __launch_bounds__(256) void device_copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                          int64_t n4, const unsigned char* __restrict__ src_tail,
                                                          unsigned char* __restrict__ dst_tail, int64_t tail) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * 4;
    int64_t i = static_cast<int64_t>(blockIdx.x) * 256 * 4 + threadIdx.x;
    for (; i + 3 * 256 < n4; i += stride) {
        float4 t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = src[i + u * 256];
#pragma unroll
        for (int u = 0; u < 4; ++u) dst[i + u * 256] = t[u];
    }
    for (; i < n4; i += 256) dst[i] = src[i];
    if (blockIdx.x == 0 && threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

int launch_device_copy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return kOk;
    const bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    if (!aligned) return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream), "copy");
    const int64_t n4 = static_cast<int64_t>(bytes / 16), tail = static_cast<int64_t>(bytes % 16);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n4, 1024), 16384));
    hipLaunchKernelGGL(device_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const float4*>(src), static_cast<float4*>(dst), n4,
                       static_cast<const unsigned char*>(src) + 16 * n4, static_cast<unsigned char*>(dst) + 16 * n4,
                       tail);
    return check_launch("copy");
}

int launch_gelu_tanh(const float* x, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(gelu_tanh_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, out, n);
    return check_launch("gelu_tanh");
}

int launch_geglu_tanh(const float* gate, const float* up, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(geglu_tanh_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, gate, up, out, n);
    return check_launch("swiglu gelu_tanh");
}

int launch_silu_backward(const float* x, const float* dy, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(silu_backward_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, dy, out, n);
    return check_launch("silu_backward");
}

int launch_gelu_tanh_backward(const float* x, const float* dy, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(gelu_tanh_backward_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, dy, out, n);
    return check_launch("gelu_tanh_backward");
}

__global__ __launch_bounds__(256) void softcap_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n,
                                                      double cap) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = static_cast<float>(cap * dtanh(static_cast<double>(x[i]) / cap));
}

__global__ __launch_bounds__(256) void sigmoid_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                      int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = static_cast<float>(dsigmoid(static_cast<double>(x[i])));
}

int launch_sigmoid(const float* x, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(sigmoid_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, out, n);
    return check_launch("sigmoid");
}

int launch_softcap(const float* x, float* out, int64_t n, double cap, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(softcap_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, out, n, cap);
    return check_launch("softcap");
}

int launch_softcap_backward(const float* x, const float* dy, float* out, int64_t n, double cap, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(softcap_backward_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, dy, out, n, cap);
    return check_launch("softcap_backward");
}

int launch_swiglu_backward(const float* gate, const float* up, const float* gate_act, const float* dproduct,
                           float* dgate, float* dup, int64_t n, hipStream_t stream, int activation) {
    if (n == 0) return kOk;
    if (activation == 1) {
        hipLaunchKernelGGL(swiglu_backward_kernel<1>, dim3(elementwise_grid(n)), dim3(256), 0, stream, gate, up,
                           gate_act, dproduct, dgate, dup, n);
        return check_launch("geglu_backward");
    }
    const int64_t n4 = aligned16({gate, up, gate_act, dproduct, dgate, dup}) ? n / 4 : 0;
    if (n4 > 0)
        hipLaunchKernelGGL(swiglu_backward4_kernel, dim3(elementwise_grid(n4)), dim3(256), 0, stream, gate, up,
                           gate_act, dproduct, dgate, dup, n4);
    const int64_t d = 4 * n4;
    if (n > d)
        hipLaunchKernelGGL(swiglu_backward_kernel<0>, dim3(elementwise_grid(n - d)), dim3(256), 0, stream, gate + d,
                           up + d, gate_act + d, dproduct + d, dgate + d, dup + d, n - d);
    return check_launch("swiglu_backward");
}

// out = (a + b) + c, elementwise in float (c may be null: a + b).
__global__ __launch_bounds__(256) void add3_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                   const float* __restrict__ c, float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float ab = a[i] + b[i];
        out[i] = c ? ab + c[i] : ab;
    }
}

int launch_add3(const float* a, const float* b, const float* c, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(add3_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, a, b, c, out, n);
    return check_launch("add3");
}

// x = f32(x * f) or f32(x / f) in place (numpy's float32 array times or over np.float32): the product or quotient
// formed in double and rounded once, which is the correctly rounded float result (a float product is exact in double;
// a double quotient of floats rounds to the float quotient, 53 >= 2 * 24 + 2 bits).
__global__ __launch_bounds__(256) void scale_kernel(float* __restrict__ x, int64_t n, float f, int divide) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const double v = static_cast<double>(x[i]);
        x[i] = static_cast<float>(divide ? v / static_cast<double>(f) : v * static_cast<double>(f));
    }
}

int launch_scale(float* x, int64_t n, float f, bool divide, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(scale_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, n, f, divide ? 1 : 0);
    return check_launch("scale");
}

int launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(add_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, a, b, out, n);
    return check_launch("add");
}

int launch_gather_rows(const float* table, const int64_t* index, float* out, int64_t rows, int64_t dim,
                       hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(rows <= 2147483647, "too many rows to gather");
    hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, table, index, out,
                       rows, dim);
    return check_launch("gather_rows");
}

}  // namespace dllm_hip
