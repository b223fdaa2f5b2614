// Softmax cross-entropy with its logit gradient (grad.hpp:395-426), and the embedding gradient (grad.hpp:431-464).
//
// Per row: the first maximum of the logits (a wave reduction with lowest-index ties); the total of
// exp(l_j - max) as one serial double chain over j ascending on one lane (a wave takes 4 rows, lane q row q's chain),
// fed by the 64 lanes in LDS chunks; the loss
// term (max + log(total)) - l[target]; then the gradient f32((e_j (1/total) - onehot) scale), fully parallel. The
// loss of a window is the serial double sum of its rows' terms in row order (negative targets skipped).
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

// Two rows per wave (measured at 8192 x 151936: 4.6 ms for the row pass against 5.6 with four rows and 6.3 with one;
// more waves per SIMD hide more of the serial chains), 512 exponentials per row and chunk (256: 5.2 ms).
constexpr int kCeRows = 2;     // rows per wave
constexpr int kCeChunk = 512;  // exponentials per row staged per pass
static_assert(kCeChunk % 256 == 0, "a chunk is whole 16-byte vectors of every lane");
constexpr int kCeLd = kCeChunk + 2;  // LDS row stride (doubles): the rows' chains read different banks

// The largest logit of row lr (math.hpp:40-53's argmax, read back as its value). Only the value enters the loss and
// the exponentials, and equal values are the same number, so which of several tied indices is taken does not matter;
// a NaN anywhere makes every exponential's total NaN, whatever the maximum. Each lane scans 16-byte vectors (eight in
// flight) when the row allows, then the lanes combine with "strictly larger wins".
__device__ inline double row_max_value(const float* lr, int64_t vocab, bool vec, int lane) {
    float best = lr[0];
    int64_t j0 = 0;
    if (vec) {
        const float4* l4 = reinterpret_cast<const float4*>(lr);
        const int64_t n4 = vocab / 4;
        int64_t q = lane;
        for (; q + 7 * 64 < n4; q += 8 * 64) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = l4[q + k * 64];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (v[k].x > best) best = v[k].x;
                if (v[k].y > best) best = v[k].y;
                if (v[k].z > best) best = v[k].z;
                if (v[k].w > best) best = v[k].w;
            }
        }
        for (; q < n4; q += 64) {
            const float4 v = l4[q];
            if (v.x > best) best = v.x;
            if (v.y > best) best = v.y;
            if (v.z > best) best = v.z;
            if (v.w > best) best = v.w;
        }
        j0 = 4 * n4;
    }
    for (int64_t j = j0 + lane; j < vocab; j += 64) {
        const float v = lr[j];
        if (v > best) best = v;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(best, off, 64);
        if (o > best) best = o;
    }
    return static_cast<double>(best);
}

// Row max + serial total + loss term for kCeRows rows per wave: all lanes form the exponentials exp(l - max) of a
// chunk of each row into LDS, then lane q adds row q's chunk onto its total in column order (16 values read ahead).
// The next chunk's logits are loaded into registers before the chains of the current one run, so the loads' latency
// hides behind the serial adds.
__global__ __launch_bounds__(64) void ce_rows_kernel(const float* __restrict__ logits, const int64_t* __restrict__ targets,
                                                     int64_t rows, int64_t vocab, double* __restrict__ row_max,
                                                     double* __restrict__ row_total, double* __restrict__ row_loss,
                                                     int* __restrict__ error_flag) {
    __shared__ __align__(16) double e[kCeRows * kCeLd];
    constexpr int kPer = kCeChunk / 64;  // logits per lane per row and chunk
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kCeRows;
    const int lane = threadIdx.x;
    const int nr = rows - r0 < kCeRows ? static_cast<int>(rows - r0) : kCeRows;
    const bool vec = vocab % 4 == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
    double mx[kCeRows];
    double my_mx = 0.0;  // lane q < nr: row r0 + q's maximum
#pragma unroll
    for (int q = 0; q < kCeRows; ++q) {
        mx[q] = 0.0;
        if (q < nr) mx[q] = row_max_value(logits + (r0 + q) * vocab, vocab, vec, lane);
        if (lane == q) my_mx = mx[q];
    }
    // Chunk c holds columns [c * kCeChunk, ...); when the rows are vector-aligned lane l loads 16-byte vectors v of
    // each row, columns 256 v + 4 l .. + 3, else columns l, l + 64, ...
    float cur[kCeRows][kPer], nxt[kCeRows][kPer];
    const auto load_chunk = [&](int64_t c0, float (&dst)[kCeRows][kPer]) {
#pragma unroll
        for (int q = 0; q < kCeRows; ++q) {
            const float* lr = logits + (r0 + (q < nr ? q : 0)) * vocab + c0;
            if (vec && c0 + kCeChunk <= vocab) {
#pragma unroll
                for (int v = 0; v < kPer / 4; ++v) {
                    const float4 a = reinterpret_cast<const float4*>(lr)[64 * v + lane];
                    dst[q][4 * v] = a.x;
                    dst[q][4 * v + 1] = a.y;
                    dst[q][4 * v + 2] = a.z;
                    dst[q][4 * v + 3] = a.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int64_t j = lane + 64 * k;
                    dst[q][k] = c0 + j < vocab ? lr[j] : 0.0f;
                }
            }
        }
    };
    // the LDS column of the k-th logit a lane holds
    const auto column = [&](int64_t c0, int k) -> int {
        if (vec && c0 + kCeChunk <= vocab) return 256 * (k / 4) + 4 * lane + (k % 4);
        return lane + 64 * k;
    };
    double total = 0.0;
    if (vocab > 0) load_chunk(0, nxt);
    for (int64_t c0 = 0; c0 < vocab; c0 += kCeChunk) {
        const int n = vocab - c0 < kCeChunk ? static_cast<int>(vocab - c0) : kCeChunk;
#pragma unroll
        for (int q = 0; q < kCeRows; ++q)
#pragma unroll
            for (int k = 0; k < kPer; ++k) cur[q][k] = nxt[q][k];
        if (c0 + kCeChunk < vocab) load_chunk(c0 + kCeChunk, nxt);
#pragma unroll
        for (int q = 0; q < kCeRows; ++q) {
            if (q >= nr) break;
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int j = column(c0, k);
                if (j < n) e[q * kCeLd + j] = dexp(static_cast<double>(cur[q][k]) - mx[q]);
            }
        }
        __syncthreads();
        if (lane < nr) {
            const double2* e2 = reinterpret_cast<const double2*>(e + lane * kCeLd);
            int j = 0;
            for (; j + 16 <= n; j += 16) {
                double2 v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = e2[j / 2 + k];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    total += v[k].x;
                    total += v[k].y;
                }
            }
            for (; j < n; ++j) total += e[lane * kCeLd + j];
        }
        __syncthreads();
    }
    if (lane < nr) {
        const int64_t r = r0 + lane;
        row_max[r] = my_mx;
        row_total[r] = total;
        const int64_t t = targets[r];
        if (t >= vocab) *error_flag = 1;
        row_loss[r] = (t >= 0 && t < vocab) ? my_mx + dlog(total) - static_cast<double>(logits[r * vocab + t]) : 0.0;
    }
}

// dlogits[r][j] = f32((exp(l - max) * (1 / total) - onehot) * scale); zeros for ignored rows. One thread takes four
// consecutive columns (16-byte loads and stores when the rows allow); the grid strides over rows.
__device__ __forceinline__ float ce_grad_value(float l, int64_t j, int64_t t, double mx, double inv, double scale) {
    const double e = dexp(static_cast<double>(l) - mx);
    const double onehot = t == j ? 1.0 : 0.0;
    return static_cast<float>((e * inv - onehot) * scale);
}

__global__ __launch_bounds__(256) void ce_grad_kernel(const float* __restrict__ logits,
                                                      const int64_t* __restrict__ targets, int64_t rows, int64_t vocab,
                                                      const double* __restrict__ row_max,
                                                      const double* __restrict__ row_total, double scale,
                                                      float* __restrict__ dlogits) {
    const int64_t j = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (j >= vocab) return;
    const bool vec = vocab % 4 == 0 && ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(dlogits)) &
                                        15) == 0;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t t = targets[r];
        const float* lr = logits + r * vocab;
        float* dr = dlogits + r * vocab;
        if (t < 0 || t >= vocab) {
            if (vec) {
                reinterpret_cast<float4*>(dr + j)[0] = float4{0.0f, 0.0f, 0.0f, 0.0f};
            } else {
                for (int k = 0; k < 4 && j + k < vocab; ++k) dr[j + k] = 0.0f;
            }
            continue;
        }
        const double mx = row_max[r];
        const double inv = 1.0 / row_total[r];
        if (vec) {
            const float4 l = reinterpret_cast<const float4*>(lr + j)[0];
            reinterpret_cast<float4*>(dr + j)[0] =
                float4{ce_grad_value(l.x, j, t, mx, inv, scale), ce_grad_value(l.y, j + 1, t, mx, inv, scale),
                       ce_grad_value(l.z, j + 2, t, mx, inv, scale), ce_grad_value(l.w, j + 3, t, mx, inv, scale)};
        } else {
            for (int k = 0; k < 4 && j + k < vocab; ++k) dr[j + k] = ce_grad_value(lr[j + k], j + k, t, mx, inv, scale);
        }
    }
}

// The loss of each segment: the serial double sum of its rows' terms in row order, negative targets skipped. One wave
// per segment: the lanes stage 512 terms at a time in LDS (+0.0 for a skipped row: the running sum starts at +0.0 and
// is never -0.0, so adding +0.0 leaves every bit as skipping does), lane 0 adds them in order.
__global__ __launch_bounds__(64) void ce_loss_kernel(const double* __restrict__ row_loss,
                                                     const int64_t* __restrict__ targets,
                                                     const int64_t* __restrict__ seg, double* __restrict__ loss_out) {
    constexpr int kStage = 512;
    __shared__ double terms[kStage];
    const int s = blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t r0 = seg[s], r1 = seg[s + 1];
    double loss = 0.0;
    for (int64_t base = r0; base < r1; base += kStage) {
        const int n = r1 - base < kStage ? static_cast<int>(r1 - base) : kStage;
        for (int i = lane; i < n; i += 64) {
            const int64_t r = base + i;
            terms[i] = targets[r] >= 0 ? row_loss[r] : 0.0;
        }
        __syncthreads();
        if (lane == 0)
            for (int i = 0; i < n; ++i) loss += terms[i];
        __syncthreads();
    }
    if (lane == 0) loss_out[s] = loss;
}

// One block per token group: out[out_row[g]] = sum of dy rows order[start[g] .. start[g + 1]) in that order.
__global__ __launch_bounds__(256) void embedding_groups_kernel(const float* __restrict__ dy, int64_t dim,
                                                               const int64_t* __restrict__ order,
                                                               const int64_t* __restrict__ start,
                                                               const int64_t* __restrict__ out_row,
                                                               float* __restrict__ out, int64_t ld_out) {
    const int64_t g = blockIdx.x;
    const int64_t s0 = start[g], s1 = start[g + 1];
    float* o = out + out_row[g] * ld_out;
    for (int64_t d = threadIdx.x; d < dim; d += 256) {
        double acc = 0.0;
        for (int64_t s = s0; s < s1; ++s) acc += static_cast<double>(dy[order[s] * dim + d]);
        o[d] = static_cast<float>(acc);
    }
}

}  // namespace

int launch_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, int64_t rows, int64_t vocab,
                         double scale, const int64_t* seg_dev, int nseg, double* row_max, double* row_total,
                         double* row_loss, double* loss_out, int* error_flag, hipStream_t stream) {
    if (rows == 0) return kOk;
    DLLM_REQUIRE(vocab > 0, "cross_entropy needs a non-empty vocabulary");
    DLLM_REQUIRE(ceil_div(rows, kCeRows) <= 0x7fffffffLL, "too many rows");
    hipLaunchKernelGGL(ce_rows_kernel, dim3(static_cast<unsigned>(ceil_div(rows, kCeRows))), dim3(64), 0, stream,
                       logits, targets, rows, vocab, row_max, row_total, row_loss, error_flag);
    DLLM_TRY(check_launch("cross_entropy rows"));
    const unsigned row_blocks = static_cast<unsigned>(rows < 65535 ? rows : 65535);
    hipLaunchKernelGGL(ce_grad_kernel, dim3(static_cast<unsigned>(ceil_div(vocab, 1024)), row_blocks), dim3(256), 0,
                       stream, logits, targets, rows, vocab, row_max, row_total, scale, dlogits);
    DLLM_TRY(check_launch("cross_entropy grad"));
    if (loss_out && nseg > 0) {
        hipLaunchKernelGGL(ce_loss_kernel, dim3(static_cast<unsigned>(nseg)), dim3(64), 0, stream, row_loss, targets,
                           seg_dev, loss_out);
        DLLM_TRY(check_launch("cross_entropy loss"));
    }
    return kOk;
}

int launch_embedding_groups(const float* dy, int64_t dim, const int64_t* order, const int64_t* start,
                            const int64_t* out_row, int64_t groups, float* out, int64_t ld_out, hipStream_t stream) {
    if (groups == 0 || dim == 0) return kOk;
    DLLM_REQUIRE(groups <= 2147483647, "too many embedding groups");
    hipLaunchKernelGGL(embedding_groups_kernel, dim3(static_cast<unsigned>(groups)), dim3(256), 0, stream, dy, dim, order,
                       start, out_row, out, ld_out);
    return check_launch("embedding_backward");
}

}  // namespace dllm_hip
