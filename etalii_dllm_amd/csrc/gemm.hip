// The matmuls of the training step, on FP64 VALU FMA with one serial accumulation per output.
//
// Every matmul of the step is C[i][j] = sum over l ascending of A[l][i] * B[l][j], accumulated in double and rounded
// to float once (cpp/include/dllm/nn.hpp:28-50 and grad.hpp:26-72 state the per-output order):
//   linear        out[r][n]  : i = r, j = n, l = k;  A = x^T (double), B = W^T (float)
//   dX            dx[r][k]   : i = r, j = k, l = n;  A = dy^T (double), B = W (float)
//   dW            dw[n][k]   : i = n, j = k, l = r;  A = dy (double),  B = x (float)
// A product of two floats is exact in double, so fma(a, b, acc) rounds exactly like the reference's multiply-then-add;
// that is the only place the library fuses a multiply and an add. The sum runs over l in one register per output, in
// ascending order, whatever the tile shape or grid: no split-K, no atomics, no cross-lane reduction, so the bits are
// independent of M, of the batch and of the CU count.
//
// Mapping to CDNA4: a wave owns 16 consecutive i (wave-uniform, so its A values come through scalar loads and are
// broadcast to all 64 lanes for free as SGPR operands of v_fma_f64) by 256 consecutive j (4 per lane, one 16-byte
// coalesced load of B per l, converted to double in registers). Per l a lane issues 64 DFMAs for one vector load
// and 4 conversions; the 4 waves of a workgroup are stacked along i and share the B row through L1/L2.
//
// Segmented mode (dW over several training windows): the l range is split into segments (one per window); each
// segment's sum is rounded to float and the per-window results are added in float in window order, the first one
// copied (trainer.py:328-332), optionally plus a per-window addend row (the tied embedding's own gradient).
#include "common.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

constexpr int kTileI = 16;     // rows per wave
constexpr int kWavesI = 4;     // waves per workgroup, stacked along i
constexpr int kTileJ = 256;    // columns per wave (4 per lane)
constexpr int kBlockI = kTileI * kWavesI;

struct GemmParams {
    const double* A;
    int64_t lda;
    const float* B;
    int64_t ldb;
    float* C;
    int64_t ldc;
    int64_t I, J;
    int64_t l0, l1;      // plain mode: the reduction range
    const int64_t* seg;  // segmented mode: nseg + 1 ascending offsets into l (device memory)
    int nseg;
    const float* bias;     // plain mode: added to the double sum before rounding
    const float* addsrc;   // plain mode: result = addsrc[i][j] + f32(sum)
    int64_t ld_add;
    const float* seg_addend;  // segmented mode: per-window addend rows
    const int* seg_addrow;    // [nseg][I]: row of seg_addend for (window, i), or -1 (adds +0.0f)
    int64_t ld_seg_add;
};

// The raw B values of row l for this lane's 4 columns. Lanes past J read a clamped in-bounds column instead (their
// sums are never stored), so the load needs no exec mask and the prefetch stays a plain register fill.
template <bool kVecB>
__device__ __forceinline__ float4 load_b(const GemmParams& p, int64_t l, int64_t j0) {
    const float* row = p.B + l * p.ldb;
    if (kVecB) {
        const int64_t j = j0 < p.J ? j0 : p.J - 4;
        return *reinterpret_cast<const float4*>(row + j);
    }
    float4 v;
    v.x = row[j0 < p.J ? j0 : p.J - 1];
    v.y = row[j0 + 1 < p.J ? j0 + 1 : p.J - 1];
    v.z = row[j0 + 2 < p.J ? j0 + 2 : p.J - 1];
    v.w = row[j0 + 3 < p.J ? j0 + 3 : p.J - 1];
    return v;
}

// One step of the reduction: converts this lane's B values of row l (loaded two steps earlier into `b`), refills
// `b` with row `l_next`, and adds the 64 products of the wave's 16 A values (one pair of scalar loads, broadcast as
// SGPR operands) and the 4 B values to their accumulators.
template <bool kVecB>
__device__ __forceinline__ void step(const GemmParams& p, const double* __restrict__ arow, float4& b, int64_t l_next,
                                     int64_t j0, double acc[kTileI][4]) {
    const double bd[4] = {b.x, b.y, b.z, b.w};
    b = load_b<kVecB>(p, l_next, j0);
#pragma unroll
    for (int q = 0; q < kTileI; ++q) {
        const double a = arow[q];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[q][c] = __builtin_fma(a, bd[c], acc[q][c]);
    }
}

// One segment's sums: acc[q][c] = sum over l in [l0, l1) of A[l][i0 + q] * B[l][j0 + c], l ascending. Unrolled by
// two with two B buffers, so each B row is requested two steps before its use and no register is copied.
template <bool kVecB>
__device__ __forceinline__ void accumulate(const GemmParams& p, int64_t i0, int64_t j0, int64_t l0, int64_t l1,
                                           double acc[kTileI][4]) {
#pragma unroll
    for (int q = 0; q < kTileI; ++q)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[q][c] = 0.0;
    if (l0 >= l1) return;
    const int64_t last = l1 - 1;
    float4 bA = load_b<kVecB>(p, l0, j0);
    float4 bB = load_b<kVecB>(p, l0 + 1 <= last ? l0 + 1 : last, j0);
    const double* __restrict__ arow = p.A + l0 * p.lda + i0;
    int64_t l = l0;
    for (; l + 1 <= last; l += 2) {
        step<kVecB>(p, arow, bA, l + 2 <= last ? l + 2 : last, j0, acc);
        step<kVecB>(p, arow + p.lda, bB, l + 3 <= last ? l + 3 : last, j0, acc);
        arow += 2 * p.lda;
    }
    if (l == last) step<kVecB>(p, arow, bA, last, j0, acc);
}

template <bool kVecB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemm_kernel(GemmParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t i0 = (static_cast<int64_t>(blockIdx.y) * kWavesI + wave) * kTileI;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * kTileJ + lane * 4;
    if (i0 >= p.I) return;  // wave-uniform
    double acc[kTileI][4];
    if (p.seg == nullptr) {
        accumulate<kVecB>(p, i0, j0, p.l0, p.l1, acc);
#pragma unroll
        for (int q = 0; q < kTileI; ++q) {
            const int64_t i = i0 + q;
            if (i >= p.I) break;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t j = j0 + c;
                if (j >= p.J) continue;
                double v = acc[q][c];
                if (p.bias) v += static_cast<double>(p.bias[j]);
                float r = static_cast<float>(v);
                if (p.addsrc) r = p.addsrc[i * p.ld_add + j] + r;
                p.C[i * p.ldc + j] = r;
            }
        }
        return;
    }
    for (int s = 0; s < p.nseg; ++s) {
        accumulate<kVecB>(p, i0, j0, p.seg[s], p.seg[s + 1], acc);
#pragma unroll
        for (int q = 0; q < kTileI; ++q) {
            const int64_t i = i0 + q;
            if (i >= p.I) break;
            const int arow = p.seg_addrow ? p.seg_addrow[static_cast<int64_t>(s) * p.I + i] : -1;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t j = j0 + c;
                if (j >= p.J) continue;
                float r = static_cast<float>(acc[q][c]);
                if (p.seg_addrow) r = r + (arow >= 0 ? p.seg_addend[arow * p.ld_seg_add + j] : 0.0f);
                float* out = p.C + i * p.ldc + j;
                *out = s == 0 ? r : *out + r;
            }
        }
    }
}

// dst[r][c] (double, row stride ldd) = src[r][c] and dstT[c][r] (double, row stride lddT) = src[r][c]; either may
// be null. Tiles of 64 x 64 through LDS so both the reads and the transposed writes are coalesced.
__global__ __launch_bounds__(256) void to_double_kernel(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                        int64_t lds, double* __restrict__ dst, int64_t ldd,
                                                        double* __restrict__ dstT, int64_t lddT) {
    __shared__ double tile[64][65];
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t r = r0 + k, c = c0 + tx;
        double v = 0.0;
        if (r < rows && c < cols) {
            v = static_cast<double>(src[r * lds + c]);
            if (dst) dst[r * ldd + c] = v;
        }
        tile[k][tx] = v;
    }
    if (!dstT) return;
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (c < cols && r < rows) dstT[c * lddT + r] = tile[tx][k];
    }
}

// dst[c][r] = src[r][c] in float (the forward pass's W^T).
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                            float* __restrict__ dst) {
    __shared__ float tile[64][65];
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t r = r0 + k, c = c0 + tx;
        tile[k][tx] = (r < rows && c < cols) ? src[r * cols + c] : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (c < cols && r < rows) dst[c * rows + r] = tile[tx][k];
    }
}

}  // namespace

int64_t padded_rows(int64_t n) { return static_cast<int64_t>(round_up(static_cast<size_t>(n > 0 ? n : 1), kBlockI)); }

int launch_gemm(const GemmCall& g, hipStream_t stream) {
    DLLM_REQUIRE(g.I >= 0 && g.J >= 0, "negative matmul size");
    DLLM_REQUIRE(g.seg == nullptr || g.nseg >= 1, "segmented matmul needs at least one segment");
    DLLM_REQUIRE(g.seg != nullptr || g.seg_addrow == nullptr, "per-window addends need segments");
    DLLM_REQUIRE(g.lda >= padded_rows(g.I), "the double operand must be padded to whole row tiles");
    if (g.I == 0 || g.J == 0) return kOk;
    GemmParams p{g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.I, g.J, g.l0, g.l1, g.seg, g.nseg, g.bias, g.addsrc,
                 g.ld_add, g.seg_addend, g.seg_addrow, g.ld_seg_add};
    const bool vec = (g.J % 4 == 0) && (g.ldb % 4 == 0) && (reinterpret_cast<uintptr_t>(g.B) % 16 == 0);
    dim3 grid(static_cast<unsigned>(ceil_div(g.J, kTileJ)), static_cast<unsigned>(ceil_div(g.I, kBlockI)));
    DLLM_REQUIRE(grid.y <= 65535u, "matmul has too many rows for one launch");
    if (vec)
        hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(256), 0, stream, p);
    return check_launch("gemm");
}

int launch_to_double(const float* src, int64_t rows, int64_t cols, int64_t lds, double* dst, int64_t ldd,
                     double* dstT, int64_t lddT, hipStream_t stream) {
    if (rows == 0 || cols == 0) return kOk;
    dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
    DLLM_REQUIRE(grid.y <= 65535u, "too many rows for one conversion launch");
    hipLaunchKernelGGL(to_double_kernel, grid, dim3(256), 0, stream, src, rows, cols, lds, dst, ldd, dstT, lddT);
    return check_launch("to_double");
}

int launch_transpose_f32(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t stream) {
    if (rows == 0 || cols == 0) return kOk;
    dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
    DLLM_REQUIRE(grid.y <= 65535u, "too many rows for one transpose launch");
    hipLaunchKernelGGL(transpose_f32_kernel, grid, dim3(256), 0, stream, src, rows, cols, dst);
    return check_launch("transpose");
}

}  // namespace dllm_hip
