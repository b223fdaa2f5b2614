// The optimizer half of the step: the global gradient norm (grad.hpp:467-473, optimizer.py:66-71 and 87-90) and the
// AdamW update (grad.hpp:481-495, optimizer.py:91-108), device-resident end to end: the clip factor is read by the
// update kernel from device memory, so no host round trip sits between the norm and the update.
//
// Each tensor's sum of squares is one serial double chain in index order (the reference's accumulation), run on one
// lane per tensor with wide loads; every tensor's chain runs concurrently. The tensor totals are then added in table
// (natural name) order on one lane, followed by sqrt and the clip factor.
#include "common.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

__device__ __forceinline__ double chain_squares(const float* __restrict__ x, int64_t n) {
    double s = 0.0;
    int64_t i = 0;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        for (; i + 4 <= n; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(x + i);
            s += static_cast<double>(v.x) * static_cast<double>(v.x);
            s += static_cast<double>(v.y) * static_cast<double>(v.y);
            s += static_cast<double>(v.z) * static_cast<double>(v.z);
            s += static_cast<double>(v.w) * static_cast<double>(v.w);
        }
    }
    for (; i < n; ++i) s += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    return s;
}

__global__ void tensor_squares_kernel(const float* __restrict__ arena, const int64_t* __restrict__ offsets,
                                      const int64_t* __restrict__ counts, int64_t tensors,
                                      double* __restrict__ per_tensor) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= tensors) return;
    per_tensor[t] = chain_squares(arena + offsets[t], counts[t]);
}

// total = sum of per_tensor in order; norm = sqrt(total); clip = max / (norm + 1e-6) when norm > max > 0, else 1.
__global__ void norm_finish_kernel(const double* __restrict__ per_tensor, int64_t tensors, double max_grad_norm,
                                   double* __restrict__ stats) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double total = 0.0;
    for (int64_t t = 0; t < tensors; ++t) total += per_tensor[t];
    const double norm = sqrt(total);
    double clip = 1.0;
    if (max_grad_norm > 0 && norm > max_grad_norm) clip = max_grad_norm / (norm + 1e-6);
    stats[0] = total;
    stats[1] = norm;
    stats[2] = clip;
}

__global__ void sum_squares_kernel(const float* __restrict__ x, int64_t n, double* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    *out = chain_squares(x, n);
}

// One element of adamw_step (grad.hpp:484-494): g = grad * scale; m, v updated and rounded to float; the parameter
// from the rounded moments.
__device__ __forceinline__ void adamw_element(float& param, float grad, float& m, float& v, double gs, double decay,
                                              const AdamWArgs& a) {
    const double g = static_cast<double>(grad) * gs;
    const float m_new = static_cast<float>(a.beta1 * static_cast<double>(m) + (1.0 - a.beta1) * g);
    const float v_new = static_cast<float>(a.beta2 * static_cast<double>(v) + (1.0 - a.beta2) * g * g);
    m = m_new;
    v = v_new;
    const double m_hat = static_cast<double>(m_new) / a.bc1;
    const double v_hat = static_cast<double>(v_new) / a.bc2;
    param = static_cast<float>(static_cast<double>(param) * decay - a.lr * m_hat / (sqrt(v_hat) + a.eps));
}

// adamw_step on chunk c = one workgroup's range [chunk_start, chunk_end) of the arena: 16-byte vectors of the four
// arrays where the range starts on one (every arena tensor does), then the range's last elements one by one.
__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ param, const float* __restrict__ grad,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    const int64_t* __restrict__ chunk_start,
                                                    const int64_t* __restrict__ chunk_end,
                                                    const double* __restrict__ chunk_decay, AdamWArgs a,
                                                    const double* __restrict__ grad_scale_dev) {
    const int64_t c = blockIdx.x;
    const int64_t i0 = chunk_start[c], i1 = chunk_end[c];
    const double gs = grad_scale_dev ? grad_scale_dev[0] : a.grad_scale;
    const double decay = 1.0 - a.lr * chunk_decay[c];
    const bool aligned = ((reinterpret_cast<uintptr_t>(param + i0) | reinterpret_cast<uintptr_t>(grad + i0) |
                           reinterpret_cast<uintptr_t>(m + i0) | reinterpret_cast<uintptr_t>(v + i0)) & 15) == 0;
    const int64_t n4 = aligned ? (i1 - i0) >> 2 : 0;
    float4* p4 = reinterpret_cast<float4*>(param + i0);
    const float4* g4 = reinterpret_cast<const float4*>(grad + i0);
    float4* m4 = reinterpret_cast<float4*>(m + i0);
    float4* v4 = reinterpret_cast<float4*>(v + i0);
    // software-pipelined: the next vector of each array is loaded before the current one is updated, so the loads'
    // latency overlaps the update's double arithmetic
    int64_t q = threadIdx.x;
    if (q < n4) {
        float4 pp = p4[q], mm = m4[q], vv = v4[q], gg = g4[q];
        for (;;) {
            const int64_t qn = q + 256;
            float4 pn, mn, vn, gn;
            if (qn < n4) {
                pn = p4[qn];
                mn = m4[qn];
                vn = v4[qn];
                gn = g4[qn];
            }
            adamw_element(pp.x, gg.x, mm.x, vv.x, gs, decay, a);
            adamw_element(pp.y, gg.y, mm.y, vv.y, gs, decay, a);
            adamw_element(pp.z, gg.z, mm.z, vv.z, gs, decay, a);
            adamw_element(pp.w, gg.w, mm.w, vv.w, gs, decay, a);
            m4[q] = mm;
            v4[q] = vv;
            p4[q] = pp;
            if (qn >= n4) break;
            q = qn;
            pp = pn;
            mm = mn;
            vv = vn;
            gg = gn;
        }
    }
    for (int64_t i = i0 + 4 * n4 + threadIdx.x; i < i1; i += 256) adamw_element(param[i], grad[i], m[i], v[i], gs, decay, a);
}

// adamw_step over one tensor of n elements (a single weight decay).
__global__ __launch_bounds__(256) void adamw_plain_kernel(float* __restrict__ param, const float* __restrict__ grad,
                                                          float* __restrict__ m, float* __restrict__ v, int64_t n,
                                                          double weight_decay, AdamWArgs a) {
    const double decay = 1.0 - a.lr * weight_decay;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const double g = static_cast<double>(grad[i]) * a.grad_scale;
        const float m_new = static_cast<float>(a.beta1 * static_cast<double>(m[i]) + (1.0 - a.beta1) * g);
        const float v_new = static_cast<float>(a.beta2 * static_cast<double>(v[i]) + (1.0 - a.beta2) * g * g);
        m[i] = m_new;
        v[i] = v_new;
        const double m_hat = static_cast<double>(m_new) / a.bc1;
        const double v_hat = static_cast<double>(v_new) / a.bc2;
        param[i] = static_cast<float>(static_cast<double>(param[i]) * decay - a.lr * m_hat / (sqrt(v_hat) + a.eps));
    }
}

}  // namespace

int launch_adamw_plain(float* param, const float* grad, float* m, float* v, int64_t n, double weight_decay,
                       const AdamWArgs& a, hipStream_t stream) {
    if (n == 0) return kOk;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(adamw_plain_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)), dim3(256), 0,
                       stream, param, grad, m, v, n, weight_decay, a);
    return check_launch("adamw");
}

int launch_global_norm(const float* arena, const int64_t* offsets, const int64_t* counts, int64_t tensors,
                       double* per_tensor, double max_grad_norm, double* stats, hipStream_t stream) {
    if (tensors > 0) {
        hipLaunchKernelGGL(tensor_squares_kernel, dim3(static_cast<unsigned>(ceil_div(tensors, 64))), dim3(64), 0,
                           stream, arena, offsets, counts, tensors, per_tensor);
        DLLM_TRY(check_launch("tensor squares"));
    }
    hipLaunchKernelGGL(norm_finish_kernel, dim3(1), dim3(64), 0, stream, per_tensor, tensors, max_grad_norm, stats);
    return check_launch("global norm");
}

int launch_norm_finish(const double* per_tensor, int64_t tensors, double max_grad_norm, double* stats,
                       hipStream_t stream) {
    hipLaunchKernelGGL(norm_finish_kernel, dim3(1), dim3(64), 0, stream, per_tensor, tensors, max_grad_norm, stats);
    return check_launch("global norm");
}

int launch_sum_squares(const float* values, int64_t n, double* result, hipStream_t stream) {
    hipLaunchKernelGGL(sum_squares_kernel, dim3(1), dim3(64), 0, stream, values, n, result);
    return check_launch("sum_squares");
}

int launch_adamw(float* param, const float* grad, float* m, float* v, const int64_t* chunk_start,
                 const int64_t* chunk_end, const double* chunk_decay, int64_t chunks, const AdamWArgs& a,
                 const double* grad_scale_dev, hipStream_t stream) {
    if (chunks == 0) return kOk;
    DLLM_REQUIRE(chunks <= 2147483647, "too many optimizer chunks");
    hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(chunks)), dim3(256), 0, stream, param, grad, m, v,
                       chunk_start, chunk_end, chunk_decay, a, grad_scale_dev);
    return check_launch("adamw");
}

}  // namespace dllm_hip
