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

constexpr int kCeRows = 4;     // rows per wave
constexpr int kCeChunk = 512;  // exponentials per row staged per pass
constexpr int kCeLd = kCeChunk + 2;  // LDS row stride (doubles): the rows' chains read different banks

// argmax (math.hpp:40-53) of row lr: the first index of the largest value. Each lane scans its own indices in
// ascending order; lanes combine by "strictly larger wins, otherwise the lower index".
__device__ inline int64_t row_argmax(const float* lr, int64_t vocab, int lane) {
    float best = 0.0f;
    int64_t bi = -1;
    for (int64_t j = lane; j < vocab; j += 64) {
        const float v = lr[j];
        if (bi < 0 || v > best) {
            best = v;
            bi = j;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int64_t oi = __shfl_xor(bi, off, 64);
        bool take;
        if (bi < 0) take = oi >= 0;
        else if (oi < 0) take = false;
        else if (ov > best) take = true;
        else if (best > ov) take = false;
        else take = oi < bi;
        if (take) {
            best = ov;
            bi = oi;
        }
    }
    return __shfl(bi, 0, 64);
}

// Row max + serial total + loss term for kCeRows rows per wave: all lanes form the exponentials exp(l - max) of a
// chunk of each row into LDS, then lane q adds row q's chunk onto its total in column order (16 values read ahead).
__global__ __launch_bounds__(64) void ce_rows_kernel(const float* __restrict__ logits, const int64_t* __restrict__ targets,
                                                     int64_t rows, int64_t vocab, double* __restrict__ row_max,
                                                     double* __restrict__ row_total, double* __restrict__ row_loss,
                                                     int* __restrict__ error_flag) {
    __shared__ __align__(16) double e[kCeRows * kCeLd];
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kCeRows;
    const int lane = threadIdx.x;
    const int nr = rows - r0 < kCeRows ? static_cast<int>(rows - r0) : kCeRows;
    double mx[kCeRows];
    double my_mx = 0.0;  // lane q < nr: row r0 + q's maximum
#pragma unroll
    for (int q = 0; q < kCeRows; ++q) {
        mx[q] = 0.0;
        if (q < nr) {
            const float* lr = logits + (r0 + q) * vocab;
            mx[q] = static_cast<double>(lr[row_argmax(lr, vocab, lane)]);
        }
        if (lane == q) my_mx = mx[q];
    }
    double total = 0.0;
    for (int64_t c0 = 0; c0 < vocab; c0 += kCeChunk) {
        const int n = vocab - c0 < kCeChunk ? static_cast<int>(vocab - c0) : kCeChunk;
#pragma unroll
        for (int q = 0; q < kCeRows; ++q) {
            if (q >= nr) break;
            const float* lr = logits + (r0 + q) * vocab + c0;
            for (int j = lane; j < n; j += 64) e[q * kCeLd + j] = dexp(static_cast<double>(lr[j]) - mx[q]);
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

// dlogits[r][j] = f32((exp(l - max) * (1 / total) - onehot) * scale); zeros for ignored rows.
__global__ __launch_bounds__(256) void ce_grad_kernel(const float* __restrict__ logits,
                                                      const int64_t* __restrict__ targets, int64_t vocab,
                                                      const double* __restrict__ row_max,
                                                      const double* __restrict__ row_total, double scale,
                                                      float* __restrict__ dlogits) {
    const int64_t r = blockIdx.y;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (j >= vocab) return;
    const int64_t t = targets[r];
    if (t < 0 || t >= vocab) {
        dlogits[r * vocab + j] = 0.0f;
        return;
    }
    const double e = dexp(static_cast<double>(logits[r * vocab + j]) - row_max[r]);
    const double inv = 1.0 / row_total[r];
    const double onehot = t == j ? 1.0 : 0.0;
    dlogits[r * vocab + j] = static_cast<float>((e * inv - onehot) * scale);
}

__global__ void ce_loss_kernel(const double* __restrict__ row_loss, const int64_t* __restrict__ targets,
                               const int64_t* __restrict__ seg, int nseg, double* __restrict__ loss_out) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    double loss = 0.0;
    for (int64_t r = seg[s]; r < seg[s + 1]; ++r)
        if (targets[r] >= 0) loss += row_loss[r];
    loss_out[s] = loss;
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
    DLLM_REQUIRE(rows <= 65535 * 1024LL, "too many rows");
    hipLaunchKernelGGL(ce_rows_kernel, dim3(static_cast<unsigned>(ceil_div(rows, kCeRows))), dim3(64), 0, stream,
                       logits, targets, rows, vocab, row_max, row_total, row_loss, error_flag);
    DLLM_TRY(check_launch("cross_entropy rows"));
    DLLM_REQUIRE(rows <= 65535, "cross_entropy launches at most 65535 rows at once");
    hipLaunchKernelGGL(ce_grad_kernel, dim3(static_cast<unsigned>(ceil_div(vocab, 256)), static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, logits, targets, vocab, row_max, row_total, scale, dlogits);
    DLLM_TRY(check_launch("cross_entropy grad"));
    if (loss_out) {
        hipLaunchKernelGGL(ce_loss_kernel, dim3(static_cast<unsigned>(ceil_div(nseg, 64))), dim3(64), 0, stream,
                           row_loss, targets, seg_dev, nseg, loss_out);
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
