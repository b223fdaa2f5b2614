// Q8_0 and Q4_0 linear layers for inference (cpp/include/dllm/quant.hpp:143-169, 355-403; kernels.cpp:310-385):
// activations quantised to Q8_0 per 32-block, the exact int32 dot of each block's 32 int8 pairs, combined per output
// as acc += (f64(xs[r][b]) f64(ws[n][b])) f64(isum_b) over blocks ascending, + bias, rounded to float once.
//
// The block dots are integer sums of at most 32 * 127 * 127 < 2^19 in magnitude: exact in any order, so they run on
// the int8 matrix cores (v_mfma_i32_16x16x32_i8, one instruction per 16 x 16 outputs and block, accumulator zero).
// The combine is the reference's double arithmetic, one multiply and one add per output and block on the vector ALU.
//
// Register layout of v_mfma_i32_16x16x32_i8 (wave64): lane L holds A[i = L % 16][k = 8 (L / 16) .. + 7] and
// B[k = 8 (L / 16) .. + 7][j = L % 16] as 8 bytes; result register r of lane L is D[4 (L / 16) + r][L % 16].
// A workgroup of 4 waves covers 64 rows x 64 outputs, a wave 32 x 32 (2 x 2 MFMA tiles); both operands are rows of
// int8 along k, so a lane's 8 bytes of a block come straight from memory.
#include "common.h"
#include "dllm_hip.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

typedef int q8_v4i __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void linear_q8_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                        const int8_t* __restrict__ wq, const float* __restrict__ ws,
                                                        const float* __restrict__ bias, float* __restrict__ out,
                                                        int64_t rows, int64_t K, int64_t N) {
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int64_t i_base = static_cast<int64_t>(blockIdx.y) * 64 + (wave >> 1) * 32;
    const int64_t n_base = static_cast<int64_t>(blockIdx.x) * 64 + (wave & 1) * 32;
    const int64_t blocks = K / 32;
    const int kq = 8 * (lane >> 4);  // this lane's bytes of a block
    // operand rows (clamped: rows past the end are read but never stored)
    const int8_t* a_row[2];
    const int8_t* b_row[2];
    for (int t = 0; t < 2; ++t) {
        const int64_t i = i_base + 16 * t + (lane & 15);
        const int64_t n = n_base + 16 * t + (lane & 15);
        a_row[t] = xq + (i < rows ? i : rows - 1) * K + kq;
        b_row[t] = wq + (n < N ? n : N - 1) * K + kq;
    }
    // the scales of this lane's outputs: rows 4 (L / 16) + r of each row tile, column L % 16 of each column tile
    const float* xs_row[2][4];
    const float* ws_row[2];
    for (int t = 0; t < 2; ++t) {
        for (int r = 0; r < 4; ++r) {
            const int64_t i = i_base + 16 * t + 4 * (lane >> 4) + r;
            xs_row[t][r] = xs + (i < rows ? i : rows - 1) * blocks;
        }
        const int64_t n = n_base + 16 * t + (lane & 15);
        ws_row[t] = ws + (n < N ? n : N - 1) * blocks;
    }
    double acc[2][2][4];
    for (int ti = 0; ti < 2; ++ti)
        for (int tj = 0; tj < 2; ++tj)
            for (int r = 0; r < 4; ++r) acc[ti][tj][r] = 0.0;
    const q8_v4i zero = {0, 0, 0, 0};
    for (int64_t b = 0; b < blocks; ++b) {
        const long a0 = *reinterpret_cast<const long*>(a_row[0] + b * 32);
        const long a1 = *reinterpret_cast<const long*>(a_row[1] + b * 32);
        const long b0 = *reinterpret_cast<const long*>(b_row[0] + b * 32);
        const long b1 = *reinterpret_cast<const long*>(b_row[1] + b * 32);
        q8_v4i isum[2][2];
        isum[0][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
        isum[0][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b1, zero, 0, 0, 0);
        isum[1][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b0, zero, 0, 0, 0);
        isum[1][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
        double wsb[2];
        for (int tj = 0; tj < 2; ++tj) wsb[tj] = static_cast<double>(ws_row[tj][b]);
        for (int ti = 0; ti < 2; ++ti)
            for (int r = 0; r < 4; ++r) {
                const double xsb = static_cast<double>(xs_row[ti][r][b]);
                for (int tj = 0; tj < 2; ++tj)
                    acc[ti][tj][r] = acc[ti][tj][r] + (xsb * wsb[tj]) * static_cast<double>(isum[ti][tj][r]);
            }
    }
    for (int ti = 0; ti < 2; ++ti)
        for (int r = 0; r < 4; ++r) {
            const int64_t i = i_base + 16 * ti + 4 * (lane >> 4) + r;
            if (i >= rows) continue;
            for (int tj = 0; tj < 2; ++tj) {
                const int64_t n = n_base + 16 * tj + (lane & 15);
                if (n >= N) continue;
                double v = acc[ti][tj][r];
                if (bias) v += static_cast<double>(bias[n]);
                out[i * N + n] = static_cast<float>(v);
            }
        }
}

// unpack_q4_0 (quant.hpp:97-108): byte j of a block holds q_j + 8 in its low and q_(j+16) + 8 in its high four bits.
__global__ __launch_bounds__(256) void unpack_q4_0_kernel(const uint8_t* __restrict__ packed, int8_t* __restrict__ out,
                                                          int64_t n) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // one packed byte
    if (e >= n / 2) return;
    const int64_t b = e / 16, j = e % 16;
    const uint8_t v = packed[e];
    out[b * 32 + j] = static_cast<int8_t>((v & 0x0F) - 8);
    out[b * 32 + j + 16] = static_cast<int8_t>((v >> 4) - 8);
}

// quantize_q4_0 (quant.hpp:67-94): one lane per block of 32.
__global__ __launch_bounds__(256) void quantize_q4_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ packed,
                                                            float* __restrict__ scales, int64_t blocks) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (b >= blocks) return;
    const float* xb = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(xb[i]);
        if (a > amax && isfinite(a)) amax = a;
    }
    const float d = amax / 7.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    scales[b] = d;
    int q[32];
    for (int i = 0; i < 32; ++i) {
        float v = 0.0f;
        if (isfinite(xb[i])) {  // round half to even (quant.hpp:28-38): floor, then the tie to the even neighbour
            const float y = xb[i] * id;
            const float f = floorf(y);
            const float diff = y - f;
            v = diff > 0.5f ? f + 1.0f : diff < 0.5f ? f : (fmodf(f, 2.0f) == 0.0f ? f : f + 1.0f);
        }
        v = v > 7.0f ? 7.0f : (v < -7.0f ? -7.0f : v);
        q[i] = static_cast<int>(v);
    }
    for (int j = 0; j < 16; ++j) packed[b * 16 + j] = static_cast<uint8_t>((q[j] + 8) | ((q[j + 16] + 8) << 4));
}

}  // namespace

int launch_linear_q8(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws, const float* bias,
                     float* out, int64_t rows, int64_t K, int64_t N, hipStream_t stream) {
    if (rows == 0 || N == 0) return kOk;
    DLLM_REQUIRE(K % 32 == 0, "Q8_0 needs in_features to be a multiple of 32");
    const dim3 grid(static_cast<unsigned>(ceil_div(N, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
    DLLM_REQUIRE(grid.y <= 65535u, "too many rows for one launch");
    hipLaunchKernelGGL(linear_q8_kernel, grid, dim3(256), 0, stream, xq, xs, wq, ws, bias, out, rows, K, N);
    return check_launch("linear_q8");
}

}  // namespace dllm_hip

using namespace dllm_hip;

extern "C" {

size_t dllm_hip_linear_q8_workspace(size_t rows, size_t in) {
    // the activations' Q8_0 values and scales; with Q4_0 weights, their unpacked int8 values follow (linear_q4)
    return round_up(rows * in, 256) + round_up(rows * (in / 32) * sizeof(float), 256);
}

size_t dllm_hip_linear_q4_workspace(size_t rows, size_t in, size_t out) {
    return dllm_hip_linear_q8_workspace(rows, in) + round_up(out * in, 256);
}

int dllm_hip_linear_q8(const float* x, const int8_t* q, const float* scales, const float* bias, float* out,
                       size_t rows, size_t in, size_t out_f, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(in % 32 == 0, "Q8_0 needs in_features to be a multiple of 32");
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_linear_q8_workspace(rows, in), "workspace too small for linear_q8");
    if (rows == 0 || out_f == 0) return kOk;
    DLLM_REQUIRE(x && q && scales && out && workspace, "null argument");
    DLLM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 8 == 0, "Q8_0 weight values must be 8-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int8_t* xq = static_cast<int8_t*>(workspace);
    float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + round_up(rows * in, 256));
    DLLM_TRY(launch_quantize_q8_0(x, xq, xs, static_cast<int64_t>(rows * in), s));
    return launch_linear_q8(xq, xs, q, scales, bias, out, static_cast<int64_t>(rows), static_cast<int64_t>(in),
                            static_cast<int64_t>(out_f), s);
}

int dllm_hip_quantize_q4_0(const float* x, uint8_t* packed, float* scales, size_t n, void* stream) {
    DLLM_REQUIRE(n % 32 == 0, "Q4_0 needs a multiple of 32 values");
    if (n == 0) return kOk;
    DLLM_REQUIRE(x && packed && scales, "null argument");
    const int64_t blocks = static_cast<int64_t>(n / 32);
    hipLaunchKernelGGL(quantize_q4_0_kernel, dim3(static_cast<unsigned>(ceil_div(blocks, 256))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, packed, scales, blocks);
    return check_launch("quantize_q4_0");
}

int dllm_hip_unpack_q4_0(const uint8_t* packed, int8_t* values, size_t n, void* stream) {
    DLLM_REQUIRE(n % 32 == 0, "Q4_0 needs a multiple of 32 values");
    if (n == 0) return kOk;
    DLLM_REQUIRE(packed && values, "null argument");
    hipLaunchKernelGGL(unpack_q4_0_kernel, dim3(static_cast<unsigned>(ceil_div(n / 2, 256))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, values, static_cast<int64_t>(n));
    return check_launch("unpack_q4_0");
}

int dllm_hip_linear_q4(const float* x, const uint8_t* q, const float* scales, const float* bias, float* out,
                       size_t rows, size_t in, size_t out_f, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(in % 32 == 0, "Q4_0 needs in_features to be a multiple of 32");
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_linear_q4_workspace(rows, in, out_f), "workspace too small for linear_q4");
    if (rows == 0 || out_f == 0) return kOk;
    DLLM_REQUIRE(x && q && scales && out && workspace, "null argument");
    int8_t* w = reinterpret_cast<int8_t*>(static_cast<char*>(workspace) + dllm_hip_linear_q8_workspace(rows, in));
    DLLM_TRY(dllm_hip_unpack_q4_0(q, w, out_f * in, stream));
    return dllm_hip_linear_q8(x, w, scales, bias, out, rows, in, out_f, workspace,
                              dllm_hip_linear_q8_workspace(rows, in), stream);
}

}  // extern "C"
