// LoRA adapters on a frozen base (src/etalii_dllm/lora.py) and the Q8_0 base quantisation (cpp/include/dllm/quant.hpp,
// src/etalii_dllm/numerics.py:106-139).
//
//   merge              W' = W + f32(linear(B, A^T)) * f32(scale)                  (lora.py:271-276)
//   adapter gradients  dA = f32(linear(B^T, dW^T)) * f32(scale),  dB = f32(linear(dW, A)) * f32(scale)  (374-383)
//   quantize_q8_0      per 32-value block: amax over the finite |x|, d = amax / 127, q = rne(x / d) clamped to
//                      +-127 (non-finite x -> 0)                                  (quant.hpp:27-60)
//   dequantize         f32(q) * d                                                 (numerics.py:138-139)
// linear(x, w)[r][n] = f32(sum over k ascending of x[r][k] w[n][k]) is the matmul of gemm.hip; the products and the
// float32 scalings are separate roundings, as the reference's numpy float32 operations.
#include <math.h>

#include "common.h"
#include "kernels.h"
#include "workspace.h"

namespace dllm_hip {

namespace {

constexpr int kQ8Block = 32;

// round half to even of |v| <= 2^22 with exact float operations (quant.hpp:27-38)
__device__ __forceinline__ float round_half_even(float v) {
    const float f = floorf(v);
    const float diff = v - f;
    if (diff > 0.5f) return f + 1.0f;
    if (diff < 0.5f) return f;
    return fmodf(f, 2.0f) == 0.0f ? f : f + 1.0f;
}

// One 32-lane half of a wave per block: the block's largest finite magnitude by lane shuffles (a maximum, so the
// order is free), then each lane its value.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                                            float* __restrict__ scales, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const bool in = i < n;
    const float xv = in ? x[i] : 0.0f;
    const float a = fabsf(xv);
    float amax = isfinite(a) ? a : 0.0f;
#pragma unroll
    for (int s = 16; s > 0; s >>= 1) {
        const float o = __shfl_xor(amax, s, kQ8Block);
        amax = o > amax ? o : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    if (!in) return;
    float v = isfinite(xv) ? round_half_even(xv * id) : 0.0f;
    v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
    q[i] = static_cast<int8_t>(v);
    if ((threadIdx.x & (kQ8Block - 1)) == 0) scales[i / kQ8Block] = d;
}

__global__ __launch_bounds__(256) void dequantize_q8_0_kernel(const int8_t* __restrict__ q,
                                                              const float* __restrict__ scales,
                                                              float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = static_cast<float>(q[i]) * scales[i / kQ8Block];
}

// out = base + x * s (float32, two roundings), or out = x * s without a base.
__global__ __launch_bounds__(256) void scale_add_kernel(const float* __restrict__ base, const float* __restrict__ x,
                                                        float s, float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float v = x[i] * s;
        out[i] = base ? base[i] + v : v;
    }
}

unsigned grid_for(int64_t n) { return static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 256), 16384)); }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

int launch_quantize_q8_0(const float* x, int8_t* q, float* scales, int64_t n, hipStream_t stream) {
    DLLM_REQUIRE(n % kQ8Block == 0, "q8_0 needs a multiple of 32 values");
    if (n == 0) return kOk;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, stream, x, q,
                       scales, n);
    return check_launch("quantize_q8_0");
}

int launch_dequantize_q8_0(const int8_t* q, const float* scales, float* out, int64_t n, hipStream_t stream) {
    DLLM_REQUIRE(n % kQ8Block == 0, "q8_0 needs a multiple of 32 values");
    if (n == 0) return kOk;
    hipLaunchKernelGGL(dequantize_q8_0_kernel, dim3(grid_for(n)), dim3(256), 0, stream, q, scales, out, n);
    return check_launch("dequantize_q8_0");
}

int launch_scale_add(const float* base, const float* x, float s, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    hipLaunchKernelGGL(scale_add_kernel, dim3(grid_for(n)), dim3(256), 0, stream, base, x, s, out, n);
    return check_launch("scale_add");
}

size_t lora_merge_workspace(int64_t out_f, int64_t in_f, int64_t rank) {
    Layout l;
    l.add<float>(static_cast<size_t>(out_f * in_f));                 // delta = linear(B, A^T)
    l.add<double>(static_cast<size_t>(rank * padded_rows(out_f)));  // B^T as double (when B cannot be read as is)
    return l.bytes;
}

int launch_lora_merge(const float* weight, const float* a, const float* b, float* out, int64_t out_f, int64_t in_f,
                      int64_t rank, float scale, void* ws, size_t ws_bytes, hipStream_t stream) {
    DLLM_REQUIRE(ws_bytes >= lora_merge_workspace(out_f, in_f, rank), "workspace too small for the LoRA merge");
    if (out_f == 0 || in_f == 0) return kOk;
    Carve c(ws, ws_bytes);
    float* delta = c.take<float>(static_cast<size_t>(out_f * in_f));
    double* bT = c.take<double>(static_cast<size_t>(rank * padded_rows(out_f)));
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    if (rank == 0) {
        DLLM_TRY(check_hip(hipMemsetAsync(delta, 0, sizeof(float) * out_f * in_f, stream), "memset"));
    } else {
        // delta[o][i] = sum over r of B[o][r] A[r][i]: matmul rows o, columns i, reduction r
        GemmCall g;
        const bool vec = in_f % 4 == 0 && aligned16(a);
        if (vec && rank % 4 == 0 && aligned16(b)) {
            g.Af = b;  // A transposed: Af[o][r]
            g.a_kind = 2;
            g.lda = rank;
        } else {
            DLLM_TRY(launch_to_double(b, out_f, rank, rank, nullptr, 0, bT, padded_rows(out_f), stream));
            g.A = bT;
            g.lda = padded_rows(out_f);
        }
        g.B = a;
        g.ldb = in_f;
        g.C = delta;
        g.ldc = in_f;
        g.I = out_f;
        g.J = in_f;
        g.l0 = 0;
        g.l1 = rank;
        DLLM_TRY(launch_gemm(g, stream));
    }
    return launch_scale_add(weight, delta, scale, out, out_f * in_f, stream);
}

size_t lora_adapter_gradients_workspace(int64_t out_f, int64_t in_f, int64_t rank) {
    Layout l;
    l.add<float>(static_cast<size_t>(in_f * rank));                  // A^T
    l.add<double>(static_cast<size_t>(out_f * padded_rows(rank)));  // B as double rows
    l.add<double>(static_cast<size_t>(in_f * padded_rows(out_f)));  // dW^T as double
    return l.bytes;
}

int launch_lora_adapter_gradients(const float* grad, const float* a, const float* b, float* da, float* db,
                                  int64_t out_f, int64_t in_f, int64_t rank, float scale, void* ws, size_t ws_bytes,
                                  hipStream_t stream) {
    DLLM_REQUIRE(ws_bytes >= lora_adapter_gradients_workspace(out_f, in_f, rank),
                 "workspace too small for the adapter gradients");
    if (rank == 0) return kOk;
    Carve c(ws, ws_bytes);
    float* aT = c.take<float>(static_cast<size_t>(in_f * rank));
    double* b_rows = c.take<double>(static_cast<size_t>(out_f * padded_rows(rank)));
    double* gT = c.take<double>(static_cast<size_t>(in_f * padded_rows(out_f)));
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    if (in_f > 0) {
        // dA[r][i] = sum over o of B[o][r] dW[o][i]: rows r, columns i, reduction o
        GemmCall g;
        const bool vec = in_f % 4 == 0 && aligned16(grad);
        if (out_f == 0) {
            DLLM_TRY(check_hip(hipMemsetAsync(da, 0, sizeof(float) * rank * in_f, stream), "memset"));
        } else {
            if (vec && rank % 4 == 0 && aligned16(b)) {
                g.Af = b;  // A rows: Af[o][r]
                g.a_kind = 1;
                g.lda = rank;
            } else {
                DLLM_TRY(launch_to_double(b, out_f, rank, rank, b_rows, padded_rows(rank), nullptr, 0, stream));
                g.A = b_rows;
                g.lda = padded_rows(rank);
            }
            g.B = grad;
            g.ldb = in_f;
            g.C = da;
            g.ldc = in_f;
            g.I = rank;
            g.J = in_f;
            g.l0 = 0;
            g.l1 = out_f;
            DLLM_TRY(launch_gemm(g, stream));
        }
        DLLM_TRY(launch_scale_add(nullptr, da, scale, da, rank * in_f, stream));
    }
    if (out_f > 0) {
        // dB[o][r] = sum over i of dW[o][i] A[r][i]: rows o, columns r, reduction i (B operand A^T [i][r])
        if (in_f == 0) {
            DLLM_TRY(check_hip(hipMemsetAsync(db, 0, sizeof(float) * out_f * rank, stream), "memset"));
        } else {
            DLLM_TRY(launch_transpose_f32(a, rank, in_f, aT, stream));
            GemmCall g;
            if (rank % 4 == 0 && in_f % 4 == 0 && aligned16(grad)) {
                g.Af = grad;  // A transposed: Af[o][i]
                g.a_kind = 2;
                g.lda = in_f;
            } else {
                DLLM_TRY(launch_to_double(grad, out_f, in_f, in_f, nullptr, 0, gT, padded_rows(out_f), stream));
                g.A = gT;
                g.lda = padded_rows(out_f);
            }
            g.B = aT;
            g.ldb = rank;
            g.C = db;
            g.ldc = rank;
            g.I = out_f;
            g.J = rank;
            g.l0 = 0;
            g.l1 = in_f;
            DLLM_TRY(launch_gemm(g, stream));
        }
        DLLM_TRY(launch_scale_add(nullptr, db, scale, db, out_f * rank, stream));
    }
    return kOk;
}

}  // namespace dllm_hip
