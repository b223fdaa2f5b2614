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
// int8 along k, so a lane's 8 bytes of a block are one 8-byte read of the LDS-staged tile.
#include "common.h"
#include "dllm_hip.h"
#include "kernels.h"
#include "lds_copy.h"

namespace dllm_hip {

namespace {

typedef int q8_v4i __attribute__((ext_vector_type(4)));

// Prefill shapes: a stage is 4 blocks (128 bytes of k). Each thread loads 2 x 16 bytes of the activation tile and
// of the weight tile (8 consecutive threads cover one row's 128 bytes) and one activation and one weight scale, into
// registers while the previous stage computes; the stage is then written to LDS (rows padded to 136 bytes: the 16
// rows a fragment read touches fall in distinct bank pairs) with the scales widened to double.
constexpr int kStageBlocks = 4;
constexpr int kLdsRow = 136;

struct Q8Stage {
    long a[2][2], b[2][2];  // two 16-byte pieces of each tile
    float xs, ws;
};

__device__ inline void q8_load_stage(Q8Stage& st, const int8_t* xq, const float* xs, const int8_t* wq,
                                     const float* ws, int64_t i0, int64_t n0, int64_t rows, int64_t K, int64_t N,
                                     int64_t b0, int tid) {
    const int64_t blocks = K / 32;
    for (int h = 0; h < 2; ++h) {
        const int c = tid + 256 * h;  // 16-byte piece: row c / 8, column c % 8
        const int row = c >> 3, col = c & 7;
        const bool valid = b0 + (col >> 1) < blocks;
        const int64_t i = i0 + row < rows ? i0 + row : rows - 1;
        const int64_t n = n0 + row < N ? n0 + row : N - 1;
        const long* pa = reinterpret_cast<const long*>(xq + i * K + b0 * 32 + col * 16);
        const long* pb = reinterpret_cast<const long*>(wq + n * K + b0 * 32 + col * 16);
        st.a[h][0] = valid ? pa[0] : 0;
        st.a[h][1] = valid ? pa[1] : 0;
        st.b[h][0] = valid ? pb[0] : 0;
        st.b[h][1] = valid ? pb[1] : 0;
    }
    const int row = tid >> 2, blk = tid & 3;  // scale entry: row tid / 4, block tid % 4 of the stage
    const bool valid = b0 + blk < blocks;
    const int64_t i = i0 + row < rows ? i0 + row : rows - 1;
    const int64_t n = n0 + row < N ? n0 + row : N - 1;
    st.xs = valid ? xs[i * blocks + b0 + blk] : 0.0f;
    st.ws = valid ? ws[n * blocks + b0 + blk] : 0.0f;
}

__global__ __launch_bounds__(256) void linear_q8_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                        const int8_t* __restrict__ wq, const float* __restrict__ ws,
                                                        const float* __restrict__ bias, float* __restrict__ out,
                                                        int64_t rows, int64_t K, int64_t N) {
    __shared__ __align__(16) int8_t a_lds[64 * kLdsRow];
    __shared__ __align__(16) int8_t b_lds[64 * kLdsRow];
    __shared__ double xs_lds[64][kStageBlocks];
    __shared__ double ws_lds[64][kStageBlocks];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * 64, n0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int wi = (wave >> 1) * 32, wj = (wave & 1) * 32;  // this wave's 32 x 32 within the tile
    const int64_t blocks = K / 32;
    const int kq = 8 * (lane >> 4);
    double acc[2][2][4];
    for (int ti = 0; ti < 2; ++ti)
        for (int tj = 0; tj < 2; ++tj)
            for (int r = 0; r < 4; ++r) acc[ti][tj][r] = 0.0;
    const q8_v4i zero = {0, 0, 0, 0};
    Q8Stage st;
    q8_load_stage(st, xq, xs, wq, ws, i0, n0, rows, K, N, 0, tid);
    for (int64_t b0 = 0; b0 < blocks; b0 += kStageBlocks) {
        lds_barrier();  // the previous stage's reads are done
        for (int h = 0; h < 2; ++h) {
            const int c = tid + 256 * h;
            const int off = (c >> 3) * kLdsRow + (c & 7) * 16;
            long* la = reinterpret_cast<long*>(a_lds + off);
            long* lb = reinterpret_cast<long*>(b_lds + off);
            la[0] = st.a[h][0];
            la[1] = st.a[h][1];
            lb[0] = st.b[h][0];
            lb[1] = st.b[h][1];
        }
        xs_lds[tid >> 2][tid & 3] = static_cast<double>(st.xs);
        ws_lds[tid >> 2][tid & 3] = static_cast<double>(st.ws);
        lds_barrier();
        if (b0 + kStageBlocks < blocks) q8_load_stage(st, xq, xs, wq, ws, i0, n0, rows, K, N, b0 + kStageBlocks, tid);
        const auto compute = [&](int blk) {
            long a[2], b[2];
            for (int t = 0; t < 2; ++t) {
                a[t] = *reinterpret_cast<const long*>(a_lds + (wi + 16 * t + (lane & 15)) * kLdsRow + blk * 32 + kq);
                b[t] = *reinterpret_cast<const long*>(b_lds + (wj + 16 * t + (lane & 15)) * kLdsRow + blk * 32 + kq);
            }
            q8_v4i isum[2][2];
            isum[0][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[0], b[0], zero, 0, 0, 0);
            isum[0][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[0], b[1], zero, 0, 0, 0);
            isum[1][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[1], b[0], zero, 0, 0, 0);
            isum[1][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[1], b[1], zero, 0, 0, 0);
            double wsb[2];
            for (int tj = 0; tj < 2; ++tj) wsb[tj] = ws_lds[wj + 16 * tj + (lane & 15)][blk];
            for (int ti = 0; ti < 2; ++ti)
                for (int r = 0; r < 4; ++r) {
                    const double xsb = xs_lds[wi + 16 * ti + 4 * (lane >> 4) + r][blk];
                    for (int tj = 0; tj < 2; ++tj)
                        acc[ti][tj][r] = acc[ti][tj][r] + (xsb * wsb[tj]) * static_cast<double>(isum[ti][tj][r]);
                }
        };
        const int nb = blocks - b0 < kStageBlocks ? static_cast<int>(blocks - b0) : kStageBlocks;
        for (int blk = 0; blk < nb; ++blk) compute(blk);
    }
    for (int ti = 0; ti < 2; ++ti)
        for (int r = 0; r < 4; ++r) {
            const int64_t i = i0 + wi + 16 * ti + 4 * (lane >> 4) + r;
            if (i >= rows) continue;
            for (int tj = 0; tj < 2; ++tj) {
                const int64_t n = n0 + wj + 16 * tj + (lane & 15);
                if (n >= N) continue;
                double v = acc[ti][tj][r];
                if (bias) v += static_cast<double>(bias[n]);
                out[i * N + n] = static_cast<float>(v);
            }
        }
}

// Decode shapes (a few rows): one wave per output n. Lane L takes blocks c + L of each chunk of 64 x kDecodeSlots
// blocks, forms the exact int32 block dot with v_dot4c_i32_i8 and the term (f64(xs) f64(ws)) f64(isum) in LDS; lane r
// then adds row r's terms over the chunk's blocks in order onto its accumulator, which is the reference's chain
// acc = acc + term_b with b ascending. A wave reads its weight row once, 64 blocks (2 KB of Q8_0, 1 KB of Q4_0) per
// load step, coalesced.
constexpr int kDecodeRows = 8;    // the largest row count that takes this kernel
constexpr int kDecodeSlots = 4;   // blocks per lane per chunk
constexpr int kDecodeChunk = 64 * kDecodeSlots;

// the block dot of 32 int8 activations with this block's weights (Q8_0: 32 int8; Q4_0: 16 bytes of packed nibbles,
// low nibble of byte j = q_j + 8, high nibble = q_(j+16) + 8, quant.hpp:97-108)
template <bool kQ4>
__device__ inline int block_dot(const int8_t* xb, const int* w) {
    const int* x = reinterpret_cast<const int*>(xb);
    int s = 0;
    if constexpr (!kQ4) {
        for (int i = 0; i < 8; ++i) s = __builtin_amdgcn_sdot4(x[i], w[i], s, false);
    } else {
        int ones = 0;
        for (int i = 0; i < 4; ++i) {
            s = __builtin_amdgcn_sdot4(x[i], w[i] & 0x0F0F0F0F, s, false);
            s = __builtin_amdgcn_sdot4(x[i + 4], (w[i] >> 4) & 0x0F0F0F0F, s, false);
            ones = __builtin_amdgcn_sdot4(x[i], 0x01010101, ones, false);
            ones = __builtin_amdgcn_sdot4(x[i + 4], 0x01010101, ones, false);
        }
        s -= 8 * ones;  // the nibbles carry q + 8
    }
    return s;
}

template <bool kQ4>
__global__ __launch_bounds__(64) void linear_q8_decode_kernel(const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xs,
                                                              const int8_t* __restrict__ wq,
                                                              const float* __restrict__ ws,
                                                              const float* __restrict__ bias, float* __restrict__ out,
                                                              int rows, int64_t K, int64_t N) {
    extern __shared__ double terms[];  // [rows][kDecodeChunk]
    constexpr int kWBytes = kQ4 ? 16 : 32;
    constexpr int kWInts = kWBytes / 4;
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t n = blockIdx.x;
    const int64_t blocks = K / 32;
    const int8_t* wrow = wq + n * blocks * kWBytes;
    const float* wsrow = ws + n * blocks;
    double acc = 0.0;
    for (int64_t c = 0; c < blocks; c += kDecodeChunk) {
        const int64_t chunk = blocks - c < kDecodeChunk ? blocks - c : kDecodeChunk;
        for (int slot = 0; slot < kDecodeSlots; ++slot) {
            const int64_t j = slot * 64 + lane;
            if (j >= chunk) break;
            const int64_t b = c + j;
            int w[kWInts];
            const long* wp = reinterpret_cast<const long*>(wrow + b * kWBytes);
            for (int i = 0; i < kWInts / 2; ++i) {
                const long v = wp[i];
                w[2 * i] = static_cast<int>(v);
                w[2 * i + 1] = static_cast<int>(v >> 32);
            }
            const double wsb = static_cast<double>(wsrow[b]);
            for (int r = 0; r < rows; ++r) {
                const int isum = block_dot<kQ4>(xq + r * K + b * 32, w);
                terms[r * kDecodeChunk + j] = (static_cast<double>(xs[r * blocks + b]) * wsb) * static_cast<double>(isum);
            }
        }
        __syncthreads();
        if (lane < rows)
            for (int64_t j = 0; j < chunk; ++j) acc = acc + terms[lane * kDecodeChunk + j];
        __syncthreads();
    }
    if (lane < rows) {
        if (bias) acc += static_cast<double>(bias[n]);
        out[lane * N + n] = static_cast<float>(acc);
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

int launch_linear_decode(bool q4, const int8_t* xq, const float* xs, const int8_t* wq, const float* ws,
                         const float* bias, float* out, int64_t rows, int64_t K, int64_t N, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(rows) * kDecodeChunk * sizeof(double);
    const auto kernel = q4 ? linear_q8_decode_kernel<true> : linear_q8_decode_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(N)), dim3(64), lds, stream, xq, xs, wq, ws, bias, out,
                       static_cast<int>(rows), K, N);
    return check_launch(q4 ? "linear_q4 decode" : "linear_q8 decode");
}

}  // namespace

int launch_linear_q8(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws, const float* bias,
                     float* out, int64_t rows, int64_t K, int64_t N, hipStream_t stream) {
    if (rows == 0 || N == 0) return kOk;
    DLLM_REQUIRE(K % 32 == 0, "Q8_0 needs in_features to be a multiple of 32");
    if (rows <= kDecodeRows && N <= 0x7FFFFFFF) {
        return launch_linear_decode(false, xq, xs, wq, ws, bias, out, rows, K, N, stream);
    }
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
    if (rows <= static_cast<size_t>(kDecodeRows) && out_f <= 0x7FFFFFFF && reinterpret_cast<uintptr_t>(q) % 8 == 0) {
        // decode shapes read the packed nibbles directly
        const hipStream_t s = static_cast<hipStream_t>(stream);
        int8_t* xq = static_cast<int8_t*>(workspace);
        float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + round_up(rows * in, 256));
        DLLM_TRY(launch_quantize_q8_0(x, xq, xs, static_cast<int64_t>(rows * in), s));
        return launch_linear_decode(true, xq, xs, reinterpret_cast<const int8_t*>(q), scales, bias, out,
                                    static_cast<int64_t>(rows), static_cast<int64_t>(in), static_cast<int64_t>(out_f),
                                    s);
    }
    int8_t* w = reinterpret_cast<int8_t*>(static_cast<char*>(workspace) + dllm_hip_linear_q8_workspace(rows, in));
    DLLM_TRY(dllm_hip_unpack_q4_0(q, w, out_f * in, stream));
    return dllm_hip_linear_q8(x, w, scales, bias, out, rows, in, out_f, workspace,
                              dllm_hip_linear_q8_workspace(rows, in), stream);
}

}  // extern "C"
