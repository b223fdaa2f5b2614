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
// Mapping to CDNA4: a wave owns 16 consecutive i (wave-uniform A values, broadcast to all 64 lanes) by 256
// consecutive j (4 per lane, converted to double in registers); per l a lane issues 64 DFMAs for one 16-byte B read
// and 4 conversions. The 4 waves of a workgroup are stacked along i. Two kernels share that mapping:
//   gemm_lds_kernel (B rows 16-byte aligned, J % 4 == 0: every matmul of the training step): the workgroup's A and
//     B tiles for 16 consecutive l are copied global -> LDS with gfx950's direct-to-LDS loads, double-buffered, so
//     the next stage is in flight during the 16 x 64 DFMAs of the current one; A is read from LDS as a broadcast.
//     Workgroups are renumbered so each XCD (own L2) gets a contiguous range of tiles, grouped 8 row blocks deep
//     so the tiles resident together share their A and B stages (fewer HBM re-reads).
//     A arrives either as doubles (A[l][i], rows padded to whole tiles) or straight from the float activations (rows
//     Af[l][i], or transposed Af[i][l]), converted to double as it is read from LDS.
//   gemm_kernel (any J and alignment): A through scalar loads as SGPR operands, B through per-lane loads.
//
// Segmented mode (dW over several training windows): the l range is split into segments (one per window); each
// segment's sum is rounded to float and the per-window results are added in float in window order, the first one
// copied (trainer.py:328-332), optionally plus a per-window addend row (the tied embedding's own gradient).
// When the tile grid is too small to fill the GPU and a scratch buffer is given, the windows run as separate
// workgroups into per-window float partials, and a second pass adds them in window order: the same roundings in
// the same order.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.h"
#include "lds_copy.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

constexpr int kTileI = 16;     // rows per wave
constexpr int kWavesI = 4;     // waves per workgroup, stacked along i
constexpr int kTileJ = 256;    // columns per wave (4 per lane)
constexpr int kBlockI = kTileI * kWavesI;
constexpr int64_t kParallelWindowsBelow = 2048;  // tiles
constexpr int64_t kGroupRows = 8;                // row blocks per L2 group
constexpr int kXcdRanges = 8;                    // XCDs (workgroups are dealt round-robin over them)
// Matrix-core launches of fewer 128 x 128 tiles take smaller ones (measured on the SmolLM2-135M step: 21.8k tokens/s
// against 12.3k with 128 x 128 tiles only; thresholds 512 and 2048 measure alike, 128 slower).
constexpr int64_t kSmallTilesBelow = 512;

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
    float* partial;  // segment-parallel mode: [nseg][I][J] per-window results (null: windows run in sequence)
    const float* Af;  // float A operands: [L][lda] (A rows) or [I][lda] (A transposed: Af[i][l] = A[l][i])
    const float* seg_weight;  // segmented mode: per-window factors on each window's result (null: none)
    const float* seg_rowscale;  // segmented mode: per-row factors on each window's result, before seg_weight
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
                if (p.seg_rowscale) r = r * p.seg_rowscale[i];  // the window's gradient unfolded
                if (p.seg_weight) r = r * p.seg_weight[s];      // the window's whole gradient times its factor
                float* out = p.C + i * p.ldc + j;
                *out = s == 0 ? r : *out + r;
            }
        }
    }
}

constexpr int kChunk = 16;      // l per LDS stage

// How A arrives: as doubles A[l][i] (rows padded to whole tiles), or straight from float activations, as rows
// Af[l][i] or transposed Af[i][l] (a row per i), converted to double when read from LDS.
enum AKind { kADouble = 0, kAFloatRows = 1, kAFloatT = 2 };

template <int kA>
struct Stage {
    // A for the stage's l and the workgroup's 64 i: [l][i] (double or float), or [i][l] (float, transposed)
    typename std::conditional<kA == kADouble, double, float>::type a[kA == kAFloatT ? kBlockI : kChunk]
                                                                     [kA == kAFloatT ? kChunk : kBlockI];
    float b[kChunk][kTileJ];  // B[l][j] for the stage's l and the workgroup's 256 j
};

// 16-byte direct-to-LDS loads per lane per stage: A (2 of doubles, 1 of floats) and B (4)
template <int kA>
constexpr int stage_loads() {
    return (kA == kADouble ? 2 : 1) + 4;
}

// Waits until at most `pending` of this wave's vector-memory operations are outstanding, then joins the workgroup.
template <int kPending>
__device__ __forceinline__ void wait_stage() {
    if (kPending == 0)
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kPending) : "memory");
}

__device__ __forceinline__ void workgroup_barrier() { asm volatile("s_barrier" ::: "memory"); }


// Issues the copies of stage rows l .. l + kChunk - 1 (rows past `last` repeat row `last`; they are never read).
// Wave w copies A rows 4w .. 4w + 3 (doubles: two rows of 64 per instruction; float rows: four rows of 64; float
// transposed: i rows 16w .. 16w + 15, 16 l each) and B rows 4w .. 4w + 3. `jl` is this lane's B column chunk.
template <int kA>
__device__ __forceinline__ void issue_stage(const GemmParams& p, Stage<kA>& st, int64_t i_blk, int64_t jl, int64_t l,
                                            int64_t last, int wave, int lane) {
    if constexpr (kA == kADouble) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int r = 4 * wave + 2 * t;
            const int64_t lr = l + r + (lane >> 5) <= last ? l + r + (lane >> 5) : last;
            copy16_to_lds(p.A + lr * p.lda + i_blk + (lane & 31) * 2, &st.a[r][0]);
        }
    } else if constexpr (kA == kAFloatRows) {
        // chunks past I (a multiple of 4) read the last chunk; their columns are never stored
        const int r = 4 * wave + (lane >> 4);
        const int64_t lr = l + r <= last ? l + r : last;
        const int64_t i = i_blk + (lane & 15) * 4 <= p.I - 4 ? i_blk + (lane & 15) * 4 : p.I - 4;
        copy16_to_lds(p.Af + lr * p.lda + i, &st.a[4 * wave][0]);
    } else {
        // rows past I read row I - 1, chunks past the row's end (l1, a multiple of 4) its last chunk: never read
        const int64_t i = i_blk + 16 * wave + (lane >> 2) < p.I ? i_blk + 16 * wave + (lane >> 2) : p.I - 1;
        const int64_t lc = l + (lane & 3) * 4 <= p.l1 - 4 ? l + (lane & 3) * 4 : p.l1 - 4;
        copy16_to_lds(p.Af + i * p.lda + lc, &st.a[16 * wave][0]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int r = 4 * wave + t;
        const int64_t lr = l + r <= last ? l + r : last;
        copy16_to_lds(p.B + lr * p.ldb + jl, &st.b[r][0]);
    }
}

// acc[Q][c] = fma(A[l][i0 + Q], b[c], acc[Q][c]) for c < 4. Lane L's `a` holds A[l][i0 + L % 16]; the DPP64
// modifier row_newbcast:Q on the FMA itself hands lane Q of each 16-lane row to the whole row, so the wave's 16 A
// values cost one 8-byte register per lane instead of 16 broadcast reads.
// A DPP instruction must come two wait states after any vector write of a register it reads, and the compiler's
// hazard checks do not look inside these statements: the first block of a row starts with s_nop 1 (after the
// conversions that produce b), and the blocks are volatile so they stay in order, each reading registers the
// block before it did not write (tests/test_dpp_hazards.py checks the built code).
template <int Q>
__device__ __forceinline__ void fma4_bcast(double (&acc)[kTileI][4], double a, const double (&b)[4]) {
    if constexpr (Q == 0)
        asm volatile("s_nop 1\n\t"
                     "v_fmac_f64_dpp %0, %4, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %1, %4, %6 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %2, %4, %7 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %3, %4, %8 row_newbcast:%9 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc[Q][0]), "+v"(acc[Q][1]), "+v"(acc[Q][2]), "+v"(acc[Q][3])
                     : "v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "n"(Q));
    else
        asm volatile("v_fmac_f64_dpp %0, %4, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %1, %4, %6 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %2, %4, %7 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_fmac_f64_dpp %3, %4, %8 row_newbcast:%9 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc[Q][0]), "+v"(acc[Q][1]), "+v"(acc[Q][2]), "+v"(acc[Q][3])
                     : "v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "n"(Q));
}

template <int Q>
__device__ __forceinline__ void fma_row(double (&acc)[kTileI][4], double a, const double (&b)[4]) {
    if constexpr (Q < kTileI) {
        fma4_bcast<Q>(acc, a, b);
        fma_row<Q + 1>(acc, a, b);
    }
}

// One stage row in registers: this lane's A value (A[l][i0 + lane % 16]) and its 4 raw B values.
struct RowOperands {
    double a;
    float4 b;
};

template <int kA>
__device__ __forceinline__ RowOperands read_row(const Stage<kA>& st, int k, int wave, int lane) {
    const int i = wave * kTileI + (lane & 15);
    double a;
    if constexpr (kA == kAFloatT)
        a = static_cast<double>(st.a[i][k]);
    else
        a = static_cast<double>(st.a[k][i]);
    return {a, *reinterpret_cast<const float4*>(&st.b[k][lane * 4])};
}

// acc[q][c] += A[l][i0 + q] * B[l][j0 + c] for one stage row.
__device__ __forceinline__ void row_fma(const RowOperands& r, double (&acc)[kTileI][4]) {
    const double bd[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    fma_row<0>(acc, r.a, bd);
}

// Rows 0 .. n-1 of a stage, l ascending; row k + 1 is read from LDS while row k's 64 FMAs run.
template <int kN, int kA>
__device__ __forceinline__ void stage_rows(const Stage<kA>& st, int n, int wave, int lane, double (&acc)[kTileI][4]) {
    if (kN > 0) {
        RowOperands cur = read_row<kA>(st, 0, wave, lane);
#pragma unroll
        for (int k = 0; k < kN; ++k) {
            RowOperands next = cur;
            if (k + 1 < kN) next = read_row<kA>(st, k + 1, wave, lane);
            row_fma(cur, acc);
            cur = next;
        }
    } else {
        for (int k = 0; k < n; ++k) row_fma(read_row<kA>(st, k, wave, lane), acc);
    }
}

// One segment's sums through the double-buffered LDS pipeline: acc[q][c] = sum over l in [l0, l1), ascending.
template <int kA>
__device__ __forceinline__ void accumulate_lds(const GemmParams& p, Stage<kA> (&st)[2], int64_t i_blk, int64_t j_blk,
                                               int wave, int lane, int64_t l0, int64_t l1, double (&acc)[kTileI][4]) {
#pragma unroll
    for (int q = 0; q < kTileI; ++q)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[q][c] = 0.0;
    if (l0 >= l1) return;
    const int64_t last = l1 - 1;
    const int64_t jl = j_blk + lane * 4 <= p.J - 4 ? j_blk + lane * 4 : p.J - 4;
    const int64_t full = (l1 - l0) / kChunk;
    const int tail = static_cast<int>((l1 - l0) % kChunk);
    const int64_t chunks = full + (tail ? 1 : 0);
    issue_stage<kA>(p, st[0], i_blk, jl, l0, last, wave, lane);
    for (int64_t c = 0; c < full; ++c) {
        if (c + 1 < chunks) {
            issue_stage<kA>(p, st[(c + 1) & 1], i_blk, jl, l0 + (c + 1) * kChunk, last, wave, lane);
            wait_stage<stage_loads<kA>()>();
        } else {
            wait_stage<0>();
        }
        stage_rows<kChunk, kA>(st[c & 1], kChunk, wave, lane, acc);
        workgroup_barrier();  // the stage is read by every wave before the next issue overwrites it
    }
    if (tail) {  // its copies were issued with the last full stage (or first, when there is none)
        wait_stage<0>();
        stage_rows<0, kA>(st[full & 1], tail, wave, lane, acc);
        workgroup_barrier();
    }
}

// Hardware workgroup id -> logical tile id such that each XCD (workgroups are dealt round-robin over the 8 XCDs)
// runs one contiguous range of tiles.
__device__ __forceinline__ int64_t xcd_contiguous(int64_t hw, int64_t n) {
    constexpr int64_t kXcds = 8;
    const int64_t q = n / kXcds, r = n % kXcds, x = hw % kXcds, k = hw / kXcds;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

enum LdsMode { kPlain = 0, kWindowsInSequence = 1, kWindowsInParallel = 2 };

// Grouped launches (kGrouped): one grid over the tiles of several independent matmuls (the experts of a layer); gx
// is then the total tile count, and a workgroup finds its matmul in the ascending tile_start table and reads that
// matmul's parameters from `groups`. The tiles of one matmul are numbered exactly as in its own launch.
template <int kMode, int kA, bool kGrouped = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemm_lds_kernel(
    GemmParams p, int64_t gx, int64_t gy, int64_t gz, const GemmParams* __restrict__ groups,
    const int64_t* __restrict__ tile_start, int ngroups) {
    __shared__ Stage<kA> st[2];
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    int64_t id;
    if constexpr (kGrouped) {
        id = xcd_contiguous(blockIdx.x, gx);
        int lo = 0, hi = ngroups - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tile_start[mid] <= id) lo = mid;
            else hi = mid - 1;
        }
        p = groups[lo];
        id -= tile_start[lo];
        gx = (p.J + kTileJ - 1) / kTileJ;
        gy = (p.I + kBlockI - 1) / kBlockI;
        gz = 1;
    } else {
        id = xcd_contiguous(blockIdx.x, gx * gy * gz);
    }
    // groups of kGroupRows row blocks x all column blocks, column-major inside a group: an XCD's resident
    // workgroups cover about 8 x 12 tiles and share their A and B stages through its L2
    const int64_t t = id % (gx * gy), bz = id / (gx * gy);
    const int64_t first = t / (kGroupRows * gx) * kGroupRows;
    const int64_t rows_in_group = gy - first < kGroupRows ? gy - first : kGroupRows;
    const int64_t by = first + (t % (kGroupRows * gx)) % rows_in_group;
    const int64_t bx = (t % (kGroupRows * gx)) / rows_in_group;
    const int64_t i_blk = by * kBlockI, j_blk = bx * kTileJ;
    const int64_t i0 = i_blk + wave * kTileI;
    const int64_t j0 = j_blk + lane * 4;
    double acc[kTileI][4];
    if (kMode == kPlain) {
        accumulate_lds<kA>(p, st, i_blk, j_blk, wave, lane, p.l0, p.l1, acc);
        if (i0 >= p.I) return;
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
    const int s_begin = kMode == kWindowsInParallel ? static_cast<int>(bz) : 0;
    const int s_end = kMode == kWindowsInParallel ? s_begin + 1 : p.nseg;
    for (int s = s_begin; s < s_end; ++s) {
        accumulate_lds<kA>(p, st, i_blk, j_blk, wave, lane, p.seg[s], p.seg[s + 1], acc);
        if (i0 >= p.I) continue;
        float* out_base = kMode == kWindowsInParallel ? p.partial + static_cast<int64_t>(s) * p.I * p.J : p.C;
        int64_t ld_out = kMode == kWindowsInParallel ? p.J : p.ldc;
        // opaque per window, so the compiler keeps no 64 output addresses live across the reduction
        asm volatile("" : "+s"(out_base), "+s"(ld_out));
#pragma unroll
        for (int q = 0; q < kTileI; ++q) {
            const int64_t i = i0 + q;
            if (i >= p.I) break;
            const int arow = p.seg_addrow ? p.seg_addrow[static_cast<int64_t>(s) * p.I + i] : -1;
            const auto out = global_ptr(out_base) + i * ld_out + j0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (j0 + c >= p.J) continue;
                float r = static_cast<float>(acc[q][c]);
                if (p.seg_addrow) r = r + (arow >= 0 ? p.seg_addend[arow * p.ld_seg_add + j0 + c] : 0.0f);
                if (p.seg_rowscale) r = r * p.seg_rowscale[i];
                if (p.seg_weight) r = r * p.seg_weight[s];
                out[c] = (kMode == kWindowsInParallel || s == 0) ? r : out[c] + r;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// FP64 matrix-core matmul (float A operands: every matmul of the training step).
//
// v_mfma_f64_16x16x4_f64 computes D[i][j] = C[i][j] + A[i][0]B[0][j] + ... + A[i][3]B[3][j] as four FMAs in
// ascending k, each rounded: exactly the serial chain acc = fma(a_l, b_l, acc) over l ascending. Issued once per 4
// consecutive l on the same accumulator, the instruction sequence is the reference's single double accumulator per
// output over l ascending, rounded to float once. The operands are floats converted to double, so every product is
// exact and each FMA rounds like the reference's multiply-then-add. Register layout (wave64): lane L supplies
// A[i = L % 16][k = L / 16] and B[k = L / 16][j = L % 16]; accumulator register r of lane L is D[L / 16 + 4r][L % 16].
//
// Padding: a stage whose l range ends inside a 4-l step feeds +0.0 in both operands for the missing l. The product is
// +0.0 and the accumulator is never -0.0 (it starts at +0.0, and a round-to-nearest sum is -0.0 only when both
// addends are), so acc + 0 == acc bit for bit, infinities and NaNs included.
//
// Mapping: a workgroup computes a (32 kBI) x (32 kBJ) tile with 4 waves in a 2 x 2 grid; a wave owns 16 kBI i x 16 kBJ
// j as kBI x kBJ MFMA blocks (8 kBI kBJ accumulator VGPRs). Stages of kMStage l of both operands are copied
// global -> LDS with direct-to-LDS loads, double-buffered; per 4-l step a wave reads kBI + kBJ fragment values from
// LDS, converts them, and issues kBI kBJ MFMAs. On gfx950 the FP64 matrix core and the vector ALU share issue cycles,
// so the copies run without vector instructions (SGPR base + fixed lane offset) and each fragment value feeds kBJ or
// kBI MFMAs: the 4 x 4 waves of the large launches spend about 6% of the matrix core's cycles on them, the 1 x 1 waves
// of the smallest grids about a quarter.
typedef double mf_v4d __attribute__((ext_vector_type(4)));
constexpr int kMStage = 32;  // l per LDS stage (the 32 x 32 tiles take twice as many: MTile::S)

// A workgroup tile of 2 x 2 waves, each wave kBI x kBJ MFMA blocks of 16 x 16: (32 kBI) x (32 kBJ) outputs. The
// step's large matmuls take 4 x 4 (128 x 128 tiles); launches whose 128 x 128 grid would leave most CUs idle take
// 2 x 2 or 1 x 1 (64 x 64, 32 x 32): the same per-output chain, more workgroups.
template <int kBI, int kBJ>
struct MTile {
    static constexpr int I = 32 * kBI;                     // workgroup tile along i
    static constexpr int J = 32 * kBJ;                     // workgroup tile along j
    // l per stage: the smallest tiles' stages are short on compute next to a copy's round trip, so they take 64
    // (c1 34.2-34.4 -> 34.0 ms per step; 128 for them, or 64 for the 64 x 64 tiles too, measured 34.8-35.0)
    static constexpr int S = kBI == 1 && kBJ == 1 ? 2 * kMStage : kMStage;
    static constexpr int PA = S * I / 4 / 256;             // 16-byte copies per thread per stage
    static constexpr int PB = S * J / 4 / 256;
    static constexpr bool swizzle = I >= 64 && J >= 64;  // the l % 4 chunk permutation needs 16 chunks a row
    static_assert(S * I % 1024 == 0 && S * J % 1024 == 0, "whole copies per thread");
};

template <int kA, int kBI, int kBJ>
struct MStage {
    float a[MTile<kBI, kBJ>::S * MTile<kBI, kBJ>::I];  // A rows: [l][i ^ 16 (l % 4)]; A transposed: [l / 4][i][l % 4]
    float b[MTile<kBI, kBJ>::S * MTile<kBI, kBJ>::J];  // A rows: [l][j ^ 16 (l % 4)]; A transposed: [l][j]
};

// Row-major stage rows of 128 floats (512 bytes) put the 4 rows a fragment read spans (l = 4s .. 4s + 3, one per
// 16 lanes) on the same LDS banks. With A read as rows (the weight gradients) row l keeps its 16-byte chunks
// XOR-permuted by 4 (l % 4): element j of row l sits at j ^ (16 (l % 4)), and a fragment read touches 64 consecutive
// banks. The copies apply the permutation through the source address each lane loads (an LDS copy's destination is
// fixed by the lane). Measured on MI355X, the permutation speeds up those matmuls by 1% and slows the transposed-A
// ones (whose A reads are already conflict-free) by 2%, so only the former use it.
template <int kA, int kBI, int kBJ>
__host__ __device__ __forceinline__ int mswizzle_chunk(int row) {
    return kA == kAFloatRows && MTile<kBI, kBJ>::swizzle ? (row & 3) << 2 : 0;
}

// The global source of copy `id` of a stage at row l, with every index clamped in bounds (rows past `last` repeat
// row `last`; their values are masked); the LDS destination of copy id is 16 * id bytes into the operand's array.
template <int kA, int kBI, int kBJ>
__host__ __device__ __forceinline__ const float* msrc_b(const GemmParams& p, int id, int64_t j_blk, int64_t l,
                                                       int64_t last) {
    constexpr int TJ = MTile<kBI, kBJ>::J;
    const int r = id / (TJ / 4), cc = (id % (TJ / 4)) ^ mswizzle_chunk<kA, kBI, kBJ>(r);
    const int64_t lr = l + r <= last ? l + r : last;
    const int64_t j = j_blk + cc * 4 <= p.J - 4 ? j_blk + cc * 4 : p.J - 4;
    return p.B + lr * p.ldb + j;
}

template <int kA, int kBI, int kBJ>
__host__ __device__ __forceinline__ const float* msrc_a(const GemmParams& p, int id, int64_t i_blk, int64_t l,
                                                       int64_t last) {
    constexpr int TI = MTile<kBI, kBJ>::I;
    if constexpr (kA == kAFloatRows) {
        const int r = id / (TI / 4), cc = (id % (TI / 4)) ^ mswizzle_chunk<kA, kBI, kBJ>(id / (TI / 4));
        const int64_t lr = l + r <= last ? l + r : last;
        const int64_t i = i_blk + cc * 4 <= p.I - 4 ? i_blk + cc * 4 : p.I - 4;
        return p.Af + lr * p.lda + i;
    } else {
        const int c = id / TI, ii = id % TI;
        const int64_t row = i_blk + ii < p.I ? i_blk + ii : p.I - 1;
        const int64_t lc = l + 4 * c <= p.l1 - 4 ? l + 4 * c : p.l1 - 4;
        return p.Af + row * p.lda + lc;
    }
}

// A stage with rows past the segment's end (the last one): every address clamped per lane.
template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void missue_stage(const GemmParams& p, MStage<kA, kBI, kBJ>& st, int64_t i_blk,
                                             int64_t j_blk, int64_t l, int64_t last, int tid) {
    using T = MTile<kBI, kBJ>;
    const int wave_base = tid & ~63;
#pragma unroll
    for (int t = 0; t < T::PB; ++t)
        copy16_to_lds(msrc_b<kA, kBI, kBJ>(p, t * 256 + tid, j_blk, l, last), &st.b[(t * 256 + wave_base) * 4]);
#pragma unroll
    for (int t = 0; t < T::PA; ++t)
        copy16_to_lds(msrc_a<kA, kBI, kBJ>(p, t * 256 + tid, i_blk, l, last), &st.a[(t * 256 + wave_base) * 4]);
}

// Steady-state copies: a stage whose rows all lie inside the segment needs no clamping along l, so each copy is a
// wave-uniform base (SGPRs, advanced per stage by scalar adds) plus this lane's fixed 32-bit byte offset, computed
// once per workgroup from the stage at l = 0. The offsets are taken from the workgroup's own block of the operands
// (B's stage rows; A's stage rows, or with A transposed the tile's first row), never from an operand's start: the
// logits' gradient that the head's dX reads transposed is 8184 x 151936 floats (4.97 GB) at the c3 bench shape,
// and offsets from its start past 2^32 bytes wrapped around.
template <int kBI, int kBJ>
struct MCopyOffsets {
    uint32_t b[MTile<kBI, kBJ>::PB], a[MTile<kBI, kBJ>::PA];
};

// Where the workgroup's A copies are measured from: the operand's start for A rows (the stage rows move the base),
// the tile's first row for A transposed (rows of the whole reduction; the base moves along l).
template <int kA>
__host__ __device__ __forceinline__ const float* a_block(const GemmParams& p, int64_t i_blk) {
    return kA == kAFloatT ? p.Af + i_blk * p.lda : p.Af;
}

template <int kA, int kBI, int kBJ>
__host__ __device__ __forceinline__ MCopyOffsets<kBI, kBJ> mcopy_offsets(const GemmParams& p, int64_t i_blk,
                                                                        int64_t j_blk, int tid) {
    using T = MTile<kBI, kBJ>;
    MCopyOffsets<kBI, kBJ> o;
    const int64_t big = int64_t{1} << 40;  // no l clamp
#pragma unroll
    for (int t = 0; t < T::PB; ++t)
        o.b[t] = static_cast<uint32_t>(
            reinterpret_cast<const char*>(msrc_b<kA, kBI, kBJ>(p, t * 256 + tid, j_blk, 0, big)) -
            reinterpret_cast<const char*>(p.B));
#pragma unroll
    for (int t = 0; t < T::PA; ++t) {
        GemmParams q = p;
        q.l1 = big;
        o.a[t] = static_cast<uint32_t>(
            reinterpret_cast<const char*>(msrc_a<kA, kBI, kBJ>(q, t * 256 + tid, i_blk, 0, big)) -
            reinterpret_cast<const char*>(a_block<kA>(p, i_blk)));
    }
    return o;
}

template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void missue_full(const GemmParams& p, MStage<kA, kBI, kBJ>& st,
                                            const MCopyOffsets<kBI, kBJ>& o, int64_t l, int wave,
                                            const float* a_base) {
    using T = MTile<kBI, kBJ>;
    const float* bb = p.B + l * p.ldb;
    const float* ab = kA == kAFloatT ? a_base + l : a_base + l * p.lda;
#pragma unroll
    for (int t = 0; t < T::PB; ++t) copy16_to_lds_s(bb, o.b[t], &st.b[(t * 256 + wave * 64) * 4]);
#pragma unroll
    for (int t = 0; t < T::PA; ++t) copy16_to_lds_s(ab, o.a[t], &st.a[(t * 256 + wave * 64) * 4]);
}

// The fragments of 4-l step s: a[q] = A[l = 4s + L/16][i = wave row base + 16q + L%16], b[q] likewise for j.
template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void mread_frags(const MStage<kA, kBI, kBJ>& st, int s, int wi, int wj, int lane,
                                            double (&a)[kBI], double (&b)[kBJ]) {
    using T = MTile<kBI, kBJ>;
    constexpr bool sw = kA == kAFloatRows && T::swizzle;
    const int k = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int q = 0; q < kBI; ++q) {
        const int i = wi * 16 * kBI + 16 * q + c16;
        if constexpr (kA == kAFloatT)
            a[q] = static_cast<double>(st.a[(s * T::I + i) * 4 + k]);
        else
            a[q] = static_cast<double>(st.a[(4 * s + k) * T::I + (sw ? (i ^ (k << 4)) : i)]);
    }
#pragma unroll
    for (int q = 0; q < kBJ; ++q) {
        const int j = wj * 16 * kBJ + 16 * q + c16;
        b[q] = static_cast<double>(st.b[(4 * s + k) * T::J + (sw ? (j ^ (k << 4)) : j)]);
    }
}

template <int kBI, int kBJ>
__device__ __forceinline__ void mfma_step(const double (&a)[kBI], const double (&b)[kBJ], mf_v4d (&acc)[kBI][kBJ]) {
#pragma unroll
    for (int bi = 0; bi < kBI; ++bi)
#pragma unroll
        for (int bj = 0; bj < kBJ; ++bj)
            acc[bi][bj] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[bi], b[bj], acc[bi][bj], 0, 0, 0);
}

// A full stage, the fragments of step s + 1 read while the MFMAs of step s run. (For the tiles of at most 2 x 2
// blocks per wave, reading the whole stage's fragments first measured slower: 1024 x 576 x 576 21.2 -> 22.0 us.)
template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void mstage_full(const MStage<kA, kBI, kBJ>& st, int wi, int wj, int lane,
                                            mf_v4d (&acc)[kBI][kBJ]) {
    using T = MTile<kBI, kBJ>;
    double a[kBI], b[kBJ];
    mread_frags<kA, kBI, kBJ>(st, 0, wi, wj, lane, a, b);
#pragma unroll
    for (int s = 0; s < T::S / 4; ++s) {
        double an[kBI], bn[kBJ];
        if (s + 1 < T::S / 4) mread_frags<kA, kBI, kBJ>(st, s + 1, wi, wj, lane, an, bn);
        mfma_step<kBI, kBJ>(a, b, acc);
        if (s + 1 < T::S / 4) {
#pragma unroll
            for (int q = 0; q < kBI; ++q) a[q] = an[q];
#pragma unroll
            for (int q = 0; q < kBJ; ++q) b[q] = bn[q];
        }
    }
}

// The last, partial stage: n < kMStage valid rows; lanes whose l is past the end feed +0.0 in both operands.
template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void mstage_tail(const MStage<kA, kBI, kBJ>& st, int n, int wi, int wj, int lane,
                                            mf_v4d (&acc)[kBI][kBJ]) {
    const int k = lane >> 4;
    for (int s = 0; 4 * s < n; ++s) {
        double a[kBI], b[kBJ];
        mread_frags<kA, kBI, kBJ>(st, s, wi, wj, lane, a, b);
        if (4 * s + k >= n) {
#pragma unroll
            for (int q = 0; q < kBI; ++q) a[q] = 0.0;
#pragma unroll
            for (int q = 0; q < kBJ; ++q) b[q] = 0.0;
        }
        mfma_step<kBI, kBJ>(a, b, acc);
    }
}

// One segment's sums: acc = sum over l in [l0, l1), ascending, through the double-buffered LDS pipeline. (Keeping
// three stages in flight instead of one measured slower for the small tiles too: their stages are bound by the LDS
// fragment reads, not by the copies.)
template <int kA, int kBI, int kBJ>
__device__ __forceinline__ void maccumulate(const GemmParams& p, MStage<kA, kBI, kBJ> (&st)[2],
                                            const MCopyOffsets<kBI, kBJ>& o, int64_t i_blk, int64_t j_blk, int tid,
                                            int wi, int wj, int lane, int64_t l0, int64_t l1,
                                            mf_v4d (&acc)[kBI][kBJ], bool primed = false, int64_t next_l0 = 0,
                                            int64_t next_l1 = 0) {
    using T = MTile<kBI, kBJ>;
#pragma unroll
    for (int bi = 0; bi < kBI; ++bi)
#pragma unroll
        for (int bj = 0; bj < kBJ; ++bj) acc[bi][bj] = mf_v4d{0.0, 0.0, 0.0, 0.0};
    if (l0 >= l1) return;
    const int64_t last = l1 - 1;
    const int64_t full = (l1 - l0) / T::S;
    const int tail = static_cast<int>((l1 - l0) % T::S);
    const int64_t chunks = full + (tail ? 1 : 0);
    const int wave = wi * 2 + wj;
    const float* a_base = a_block<kA>(p, i_blk);  // the copies' A base, once per tile
    auto issue = [&](MStage<kA, kBI, kBJ>& buf, int64_t l, int64_t end) {
        if (l + T::S <= end) missue_full<kA, kBI, kBJ>(p, buf, o, l, wave, a_base);
        else missue_stage<kA, kBI, kBJ>(p, buf, i_blk, j_blk, l, end - 1, tid);
    };
    if (!primed) issue(st[0], l0, l1);
    for (int64_t c = 0; c < full; ++c) {
        if (c + 1 < chunks) {
            issue(st[(c + 1) & 1], l0 + (c + 1) * T::S, l1);
            wait_stage<T::PA + T::PB>();  // this stage landed; the next one's copies in flight
        } else {
            wait_stage<0>();
        }
        mstage_full<kA, kBI, kBJ>(st[c & 1], wi, wj, lane, acc);
        // every wave has issued its reads of the stage before the next issue overwrites it. The compiler places the
        // stage's last MFMAs, and the waits for their fragment reads, after this barrier; those reads are already in
        // the CU's LDS pipeline, and the copy that refills the buffer is issued after the barrier and writes only
        // when its data returns from memory. (Waiting for the reads here cost 0.45% of the c3 step.)
        workgroup_barrier();
    }
    if (tail) {
        wait_stage<0>();
        mstage_tail<kA, kBI, kBJ>(st[full & 1], tail, wi, wj, lane, acc);
        workgroup_barrier();
    }
    // the next window's first stage (both buffers are free after the last barrier): its copies fly during this
    // window's epilogue
    if (next_l0 < next_l1) issue(st[0], next_l0, next_l1);
}

template <int kMode, int kA, bool kGrouped = false, int kBI = 4, int kBJ = 4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, kBI * kBJ >= 16 ? 2 : 4))) void
gemm_mfma_kernel(GemmParams p, int64_t gx, int64_t gy, int64_t gz, const GemmParams* __restrict__ groups,
                 const int64_t* __restrict__ tile_start, int ngroups) {
    using T = MTile<kBI, kBJ>;
    __shared__ MStage<kA, kBI, kBJ> st[2];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wi = wave >> 1, wj = wave & 1;
    int64_t id;
    if constexpr (kGrouped) {
        // the XCD ranges follow the tile starts of the table (gy: its capacity); workgroups past their XCD's range
        // have no tile
        const int64_t* xcd_first = tile_start + gy + 1;
        const int64_t x = blockIdx.x % kXcdRanges;
        id = xcd_first[x] + blockIdx.x / kXcdRanges;
        if (id >= xcd_first[x + 1]) return;
        int lo = 0, hi = ngroups - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tile_start[mid] <= id) lo = mid;
            else hi = mid - 1;
        }
        p = groups[lo];
        id -= tile_start[lo];
        gx = (p.J + T::J - 1) / T::J;
        gy = (p.I + T::I - 1) / T::I;
        gz = 1;
    } else {
        id = xcd_contiguous(blockIdx.x, gx * gy * gz);
    }
    // groups of kGroupRows row blocks x all column blocks, column-major inside a group (L2 reuse on one XCD)
    const int64_t t = id % (gx * gy), bz = id / (gx * gy);
    const int64_t first = t / (kGroupRows * gx) * kGroupRows;
    const int64_t rows_in_group = gy - first < kGroupRows ? gy - first : kGroupRows;
    const int64_t by = first + (t % (kGroupRows * gx)) % rows_in_group;
    const int64_t bx = (t % (kGroupRows * gx)) / rows_in_group;
    const int64_t i_blk = by * T::I, j_blk = bx * T::J;
    const int64_t iw = i_blk + wi * 16 * kBI;  // this wave's first row
    const int64_t jw = j_blk + wj * 16 * kBJ + (lane & 15);
    const int ri = lane >> 4;
    const MCopyOffsets<kBI, kBJ> o = mcopy_offsets<kA, kBI, kBJ>(p, i_blk, j_blk, tid);
    mf_v4d acc[kBI][kBJ];
    if (kMode == kPlain) {
        maccumulate<kA, kBI, kBJ>(p, st, o, i_blk, j_blk, tid, wi, wj, lane, p.l0, p.l1, acc);
        if (iw >= p.I) return;
        // Per row block bi, the loads (bias, addend) are issued before the block's stores: interleaved, each store
        // could alias the next load and serialise the memory round trips. The addend is either the output itself
        // (same rows) or disjoint from it, so reading it first gives the same values.
        const auto C = global_ptr(p.C);
        const auto bias = global_ptr(p.bias);
        const auto addsrc = global_ptr(p.addsrc);
#pragma unroll
        for (int bi = 0; bi < kBI; ++bi) {
            float val[4][kBJ];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t i = iw + 16 * bi + ri + 4 * r;
                const int64_t ic = i < p.I ? i : p.I - 1;
#pragma unroll
                for (int bj = 0; bj < kBJ; ++bj) {
                    const int64_t j = jw + 16 * bj;
                    const int64_t jc = j < p.J ? j : p.J - 1;
                    double v = acc[bi][bj][r];
                    if (p.bias) v += static_cast<double>(bias[jc]);
                    float out = static_cast<float>(v);
                    if (p.addsrc) out = addsrc[ic * p.ld_add + jc] + out;
                    val[r][bj] = out;
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t i = iw + 16 * bi + ri + 4 * r;
                if (i >= p.I) continue;
#pragma unroll
                for (int bj = 0; bj < kBJ; ++bj) {
                    const int64_t j = jw + 16 * bj;
                    if (j < p.J) C[i * p.ldc + j] = val[r][bj];
                }
            }
        }
        return;
    }
    const int s_begin = kMode == kWindowsInParallel ? static_cast<int>(bz) : 0;
    const int s_end = kMode == kWindowsInParallel ? s_begin + 1 : p.nseg;
    const auto seg = global_ptr(p.seg);
    // windows in sequence: each window's reduction issues the next one's first stage before this epilogue
    bool primed = false;
    for (int s = s_begin; s < s_end; ++s) {
        const int64_t l0 = seg[s], l1 = seg[s + 1];
        const int64_t n0 = s + 1 < s_end && l0 < l1 ? seg[s + 1] : 0, n1 = s + 1 < s_end && l0 < l1 ? seg[s + 2] : 0;
        maccumulate<kA, kBI, kBJ>(p, st, o, i_blk, j_blk, tid, wi, wj, lane, l0, l1, acc, primed, n0, n1);
        primed = n0 < n1;
        if (iw >= p.I) continue;
        float* out_base = kMode == kWindowsInParallel ? p.partial + static_cast<int64_t>(s) * p.I * p.J : p.C;
        int64_t ld_out = kMode == kWindowsInParallel ? p.J : p.ldc;
        asm volatile("" : "+s"(out_base), "+s"(ld_out));
        const auto out_g = global_ptr(out_base);
        // Per row block bi, every load of the epilogue (the running sum of the earlier windows, the addend rows, the
        // row factors) is issued before the block's first store, each kind unconditionally or under one uniform
        // branch: a load under a per-element branch, or next to a store that could alias it, costs a whole memory
        // round trip per element.
        const bool add_to_out = kMode == kWindowsInSequence && s > 0;
        const float wscale = p.seg_weight ? global_ptr(p.seg_weight)[s] : 1.0f;
        const auto seg_addrow = global_ptr(p.seg_addrow);
        const auto seg_addend = global_ptr(p.seg_addend);
        const auto seg_rowscale = global_ptr(p.seg_rowscale);
        // the row and column of this lane, opaque per window: their many derived addresses are recomputed here
        // rather than kept (or spilled) across the reduction
        int64_t iw_e = iw, jw_e = jw;
        asm volatile("" : "+s"(iw_e), "+v"(jw_e));
#pragma unroll
        for (int bi = 0; bi < kBI; ++bi) {
            int64_t ic[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t i = iw_e + 16 * bi + ri + 4 * r;
                ic[r] = i < p.I ? i : p.I - 1;
            }
            int64_t jc[kBJ];
#pragma unroll
            for (int bj = 0; bj < kBJ; ++bj) {
                const int64_t j = jw_e + 16 * bj;
                jc[bj] = j < p.J ? j : p.J - 1;
            }
            float run[4][kBJ];  // read even for the first window (unused there): no branch around the loads
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int bj = 0; bj < kBJ; ++bj) run[r][bj] = out_g[ic[r] * ld_out + jc[bj]];
            float addend[4][kBJ];
            if (p.seg_addrow) {
                int arow[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) arow[r] = seg_addrow[static_cast<int64_t>(s) * p.I + ic[r]];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int bj = 0; bj < kBJ; ++bj) {  // row 0 stands in for "no addend" (loaded, then dropped)
                        const float a = seg_addend[(arow[r] >= 0 ? arow[r] : 0) * p.ld_seg_add + jc[bj]];
                        addend[r][bj] = arow[r] >= 0 ? a : 0.0f;
                    }
            }
            float rscale[4];
            if (p.seg_rowscale) {
#pragma unroll
                for (int r = 0; r < 4; ++r) rscale[r] = seg_rowscale[ic[r]];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t i = iw_e + 16 * bi + ri + 4 * r;
                if (i >= p.I) continue;
                const auto out = out_g + i * ld_out;
#pragma unroll
                for (int bj = 0; bj < kBJ; ++bj) {
                    const int64_t j = jw_e + 16 * bj;
                    if (j >= p.J) continue;
                    float v = static_cast<float>(acc[bi][bj][r]);
                    if (p.seg_addrow) v = v + addend[r][bj];
                    if (p.seg_rowscale) v = v * rscale[r];  // the window's gradient unfolded (RoPE attention factor)
                    if (p.seg_weight) v = v * wscale;       // the window's whole gradient times its factor
                    out[j] = add_to_out ? run[r][bj] + v : v;
                }
            }
        }
    }
}

// C[i][j] = partial[0][i][j] + partial[1][i][j] + ... in float, window order (trainer.py:328-332).
// Contiguous output (ldc == J, 16-byte aligned, I J % 4 == 0): four elements per thread, the windows' loads issued
// eight at a time ahead of the adds, which stay in window order.
__global__ __launch_bounds__(256) void window_sum4_kernel(const float4* __restrict__ partial, int64_t n4, int nseg,
                                                          float4* __restrict__ C) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n4;
         e += static_cast<int64_t>(gridDim.x) * 256) {
        float4 t = partial[e];
        for (int s0 = 1; s0 < nseg; s0 += 8) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (s0 + k < nseg) v[k] = partial[static_cast<int64_t>(s0 + k) * n4 + e];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (s0 + k < nseg) {
                    t.x = t.x + v[k].x;
                    t.y = t.y + v[k].y;
                    t.z = t.z + v[k].z;
                    t.w = t.w + v[k].w;
                }
        }
        C[e] = t;
    }
}

__global__ __launch_bounds__(256) void window_sum_kernel(const float* __restrict__ partial, int64_t I, int64_t J,
                                                         int nseg, float* __restrict__ C, int64_t ldc) {
    const int64_t n = I * J;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * 256) {
        float t = partial[e];
        for (int s = 1; s < nseg; ++s) t = t + partial[static_cast<int64_t>(s) * n + e];
        C[(e / J) * ldc + e % J] = t;
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

// Many transposes in one launch: workgroup -> job through the ascending tile-start table, then one 64 x 64 tile.
__global__ __launch_bounds__(256) void transpose_batch_kernel(const TransposeJob* __restrict__ jobs,
                                                              const int64_t* __restrict__ tile_start, int njobs) {
    __shared__ float tile[64][65];
    const int64_t id = blockIdx.x;
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= id) lo = mid;
        else hi = mid - 1;
    }
    const TransposeJob jb = jobs[lo];
    const int64_t t = id - tile_start[lo];
    const int64_t tiles_c = (jb.cols + 63) / 64;
    const int64_t r0 = t / tiles_c * 64, c0 = t % tiles_c * 64;
    if (jb.rows % 4 == 0 && jb.cols % 4 == 0 &&
        ((reinterpret_cast<uintptr_t>(jb.src) | reinterpret_cast<uintptr_t>(jb.dst)) & 15) == 0) {
        // 16-byte vectors both ways: thread (row k, column group g) reads src[r0 + k][c0 + 4g .. + 3], then writes
        // dst[c0 + k][r0 + 4g .. + 3]; with both sizes multiples of 4 a vector is wholly inside or outside
        const int g = threadIdx.x & 15, k0 = threadIdx.x >> 4;
        for (int k = k0; k < 64; k += 16) {
            const int64_t r = r0 + k, c = c0 + 4 * g;
            float4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (r < jb.rows && c < jb.cols) v = *reinterpret_cast<const float4*>(jb.src + r * jb.cols + c);
            tile[k][4 * g] = v.x;
            tile[k][4 * g + 1] = v.y;
            tile[k][4 * g + 2] = v.z;
            tile[k][4 * g + 3] = v.w;
        }
        __syncthreads();
        for (int k = k0; k < 64; k += 16) {
            const int64_t c = c0 + k, r = r0 + 4 * g;
            if (c < jb.cols && r < jb.rows)
                *reinterpret_cast<float4*>(jb.dst + c * jb.rows + r) =
                    float4{tile[4 * g][k], tile[4 * g + 1][k], tile[4 * g + 2][k], tile[4 * g + 3][k]};
        }
        return;
    }
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t r = r0 + k, c = c0 + tx;
        tile[k][tx] = (r < jb.rows && c < jb.cols) ? jb.src[r * jb.cols + c] : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (c < jb.cols && r < jb.rows) jb.dst[c * jb.rows + r] = tile[tx][k];
    }
}

}  // namespace

int64_t padded_rows(int64_t n) { return static_cast<int64_t>(round_up(static_cast<size_t>(n > 0 ? n : 1), kBlockI)); }

namespace {

// Whether the matrix-core kernel's 32-bit per-lane copy offsets reach every element of a workgroup's block: 128 A
// rows (transposed) or a stage's rows of A and B (at most 64), from the block's base.
bool mfma_offsets_fit(const GemmCall& g) {
    constexpr int64_t kLimit = int64_t{1} << 32;
    const int64_t a = g.a_kind == kAFloatT ? 128 * g.lda : 2 * kMStage * g.lda + g.I;
    return 4 * a < kLimit && 4 * (2 * kMStage * g.ldb + g.J) < kLimit;
}

// Whether a float-A call fits the matrix-core kernel's 16-byte staging (the conditions launch_gemm requires).
bool mfma_shape(const GemmCall& g) {
    const bool vec = g.J % 4 == 0 && g.ldb % 4 == 0 && reinterpret_cast<uintptr_t>(g.B) % 16 == 0;
    if (!vec || g.lda % 4 != 0 || reinterpret_cast<uintptr_t>(g.Af) % 16 != 0) return false;
    if (!mfma_offsets_fit(g)) return false;
    if (g.a_kind == kAFloatRows) return g.I % 4 == 0 && g.lda >= g.I;
    return g.seg == nullptr && g.l0 == 0 && g.l1 % 4 == 0 && g.l1 >= 4 && g.lda >= g.l1;
}

GemmParams params_of(const GemmCall& g) {
    return GemmParams{g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.I, g.J, g.l0, g.l1, g.seg, g.nseg, g.bias, g.addsrc,
                      g.ld_add, g.seg_addend, g.seg_addrow, g.ld_seg_add, nullptr, g.Af, g.seg_weight,
                      g.seg_rowscale};
}

}  // namespace

bool gemm_mfma_shape(const GemmCall& g) { return g.a_kind != kADouble && mfma_shape(g); }

// The table: GemmParams[capacity], then the tile starts (capacity + 1), then the first tile of each XCD's range (9).
size_t gemm_group_bytes(int n) {
    return round_up(sizeof(GemmParams) * static_cast<size_t>(n), 8) +
           sizeof(int64_t) * (static_cast<size_t>(n) + 1 + kXcdRanges + 1);
}

int gemm_group_prepare(const GemmCall* calls, int n, int capacity, void* host_table, GemmGroup* group) {
    DLLM_REQUIRE(n >= 1 && n <= capacity, "a matmul group needs between one and `capacity` matmuls");
    const int ak = calls[0].a_kind;
    const bool seg = calls[0].seg != nullptr;
    DLLM_REQUIRE(ak == kAFloatRows || ak == kAFloatT, "grouped matmuls read float A operands");
    GemmParams* ps = static_cast<GemmParams*>(host_table);
    int64_t* starts = reinterpret_cast<int64_t*>(static_cast<char*>(host_table) +
                                                 round_up(sizeof(GemmParams) * static_cast<size_t>(capacity), 8));
    // plain groups whose 128 x 128 tiles would leave most CUs idle take 64 x 64 or 32 x 32 ones (as launch_gemm)
    int tile = 4;
    if (!seg) {
        while (tile > 1) {
            int64_t count = 0;
            for (int k = 0; k < n; ++k)
                count += ceil_div(calls[k].J, 32 * tile) * ceil_div(calls[k].I, 32 * tile);
            if (count >= kSmallTilesBelow) break;
            tile /= 2;
        }
    }
    int64_t tiles = 0;
    int used = 0;
    for (int k = 0; k < n; ++k) {
        const GemmCall& g = calls[k];
        DLLM_REQUIRE(g.a_kind == ak && (g.seg != nullptr) == seg, "the matmuls of a group share their mode");
        DLLM_REQUIRE(g.seg_addrow == nullptr && g.seg_partial == nullptr, "grouped matmuls take no window addends");
        DLLM_REQUIRE(mfma_offsets_fit(g), "matmul operand rows too long for the matrix-core kernel's copy offsets");
        DLLM_REQUIRE(g.J % 4 == 0 && g.ldb % 4 == 0 && reinterpret_cast<uintptr_t>(g.B) % 16 == 0,
                     "float A operands need B rows of whole 16-byte chunks");
        DLLM_REQUIRE(g.lda % 4 == 0 && reinterpret_cast<uintptr_t>(g.Af) % 16 == 0,
                     "float A rows must be 16-byte aligned");
        if (ak == kAFloatRows) DLLM_REQUIRE(g.I % 4 == 0 && g.lda >= g.I, "float A rows must hold whole chunks of I");
        if (ak == kAFloatT)
            DLLM_REQUIRE(!seg && g.l0 == 0 && g.l1 % 4 == 0 && g.l1 >= 4 && g.lda >= g.l1,
                         "transposed float A needs a plain reduction over whole 16-byte chunks");
        if (g.I == 0 || g.J == 0) continue;
        ps[used] = params_of(g);
        starts[used] = tiles;
        tiles += static_cast<int64_t>(ceil_div(g.J, 32 * tile) * ceil_div(g.I, 32 * tile));
        ++used;
    }
    starts[used] = tiles;
    DLLM_REQUIRE(tiles < (int64_t{1} << 31), "matmul group too large for one launch");
    // Each XCD takes a contiguous range of tiles (its L2 serves the A and B blocks they share) holding an equal share
    // of the work. A tile's work is its reduction length plus a fixed cost; the tiles of the experts' weight
    // gradients all have the size of the output, so equal tile counts would load an XCD by the rows of its experts.
    int64_t* xcd_first = starts + capacity + 1;
    {
        std::vector<double> work(static_cast<size_t>(used));
        double total = 0.0;
        for (int k = 0; k < used; ++k) {
            const GemmParams& q = ps[k];
            work[static_cast<size_t>(k)] = static_cast<double>(q.l1 - q.l0) + 64.0;
            total += work[static_cast<size_t>(k)] * static_cast<double>(starts[k + 1] - starts[k]);
        }
        int64_t longest = 0;
        int k = 0;
        double before = 0.0;  // work of the tiles ahead of group k
        xcd_first[0] = 0;
        for (int x = 1; x <= kXcdRanges; ++x) {
            if (x == kXcdRanges) {
                xcd_first[x] = tiles;
            } else {
                const double target = total * x / kXcdRanges;
                while (k < used && before + work[static_cast<size_t>(k)] * (starts[k + 1] - starts[k]) <= target) {
                    before += work[static_cast<size_t>(k)] * static_cast<double>(starts[k + 1] - starts[k]);
                    ++k;
                }
                int64_t t = k < used ? starts[k] + static_cast<int64_t>((target - before) / work[static_cast<size_t>(k)])
                                     : tiles;
                xcd_first[x] = std::min(std::max(t, xcd_first[x - 1]), tiles);
            }
            longest = std::max(longest, xcd_first[x] - xcd_first[x - 1]);
        }
        group->grid = longest * kXcdRanges;
    }
    group->count = used;
    group->tile = tile;
    group->tiles = tiles;
    group->a_kind = ak;
    group->segmented = seg ? 1 : 0;
    group->capacity = capacity;
    return kOk;
}

// ---- row groups: the matmuls of a group take consecutive row ranges of shared operands, known on the device ----
//
// The routed experts' matmuls: matmul k reads and writes rows [start[k], start[k + 1]) of the grouped operands
// (start in device memory, from the grouping kernels), so its row count and operand addresses are only known on the
// device. The host lays out a template table once (every matmul at row 0 with no rows); before each launch a
// one-workgroup kernel writes the live table from it: operand addresses advanced by the start times each operand's
// row stride, the row count as I (plain) or as the reduction length (segmented), the tile starts and the XCD ranges
// of equal work, each at most `cap` tiles so that the host's grid (8 cap workgroups) covers every tile.

namespace {

__global__ __launch_bounds__(256) void gemm_row_group_fill_kernel(const GemmParams* __restrict__ templ,
                                                                  GemmParams* __restrict__ table, int n,
                                                                  int capacity, const int64_t* __restrict__ start,
                                                                  GemmRowShift shift, int tile, int64_t cap) {
    constexpr int kMaxGroup = 1024;
    __shared__ int64_t ntiles[kMaxGroup];
    __shared__ double nwork[kMaxGroup];
    int64_t* starts = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(table) +
                                                 ((sizeof(GemmParams) * static_cast<size_t>(capacity) + 7) & ~size_t{7}));
    int64_t* xcd_first = starts + capacity + 1;
    for (int k = threadIdx.x; k < n; k += 256) {
        GemmParams q = templ[k];
        const int64_t st = start[k], rows = start[k + 1] - st;
        q.Af += st * shift.a;
        q.B += st * shift.b;
        q.C += st * shift.c;
        if (q.addsrc) q.addsrc += st * shift.add;
        if (shift.rows_in_reduction) q.l1 = rows;
        else q.I = rows;
        table[k] = q;
        ntiles[k] = q.I > 0 && q.J > 0 ? ((q.J + 32 * tile - 1) / (32 * tile)) * ((q.I + 32 * tile - 1) / (32 * tile)) : 0;
        nwork[k] = static_cast<double>(q.l1 - q.l0) + 64.0;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    int64_t tiles = 0;
    double total = 0.0;
    for (int k = 0; k < n; ++k) {
        starts[k] = tiles;
        tiles += ntiles[k];
        total += nwork[k] * static_cast<double>(ntiles[k]);
    }
    starts[n] = tiles;
    // XCD x takes tiles [xcd_first[x], xcd_first[x + 1]): cut at equal shares of the work, each range at most cap
    // tiles and the ranges left able to hold the tiles left
    xcd_first[0] = 0;
    int k = 0;
    double before = 0.0;
    for (int x = 1; x <= kXcdRanges; ++x) {
        int64_t t = tiles;
        if (x < kXcdRanges) {
            const double target = total * x / kXcdRanges;
            while (k < n && before + nwork[k] * static_cast<double>(ntiles[k]) <= target) {
                before += nwork[k] * static_cast<double>(ntiles[k]);
                ++k;
            }
            t = k < n ? starts[k] + static_cast<int64_t>((target - before) / nwork[k]) : tiles;
        }
        const int64_t lo = xcd_first[x - 1];
        t = t < lo ? lo : t;
        t = t > lo + cap ? lo + cap : t;                             // this range at most cap tiles
        const int64_t need = tiles - cap * (kXcdRanges - x);         // the later ranges hold the rest
        t = t < need ? need : t;
        xcd_first[x] = t > tiles ? tiles : t;
    }
}

}  // namespace

int gemm_row_group_prepare(const GemmCall* calls, int n, int capacity, int tile, int64_t max_tiles, void* host_table,
                           GemmGroup* group) {
    DLLM_REQUIRE(n >= 1 && n <= capacity && capacity <= 1024, "a row group holds 1 to 1024 matmuls");
    const int ak = calls[0].a_kind;
    const bool seg = calls[0].seg != nullptr;
    DLLM_REQUIRE(ak == kAFloatRows || ak == kAFloatT, "grouped matmuls read float A operands");
    DLLM_REQUIRE(tile == 4 || (!seg && (tile == 2 || tile == 1)), "row groups take 128 tiles, or plain 64 or 32");
    GemmParams* ps = static_cast<GemmParams*>(host_table);
    for (int k = 0; k < n; ++k) {
        const GemmCall& g = calls[k];
        DLLM_REQUIRE(g.a_kind == ak && (g.seg != nullptr) == seg, "the matmuls of a group share their mode");
        DLLM_REQUIRE(g.seg_addrow == nullptr && g.seg_partial == nullptr, "grouped matmuls take no window addends");
        DLLM_REQUIRE(mfma_offsets_fit(g), "matmul operand rows too long for the matrix-core kernel's copy offsets");
        DLLM_REQUIRE(g.J % 4 == 0 && g.ldb % 4 == 0 && g.lda % 4 == 0 && reinterpret_cast<uintptr_t>(g.B) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(g.Af) % 16 == 0,
                     "row groups need operand rows of whole 16-byte chunks");
        if (ak == kAFloatRows) DLLM_REQUIRE(g.I % 4 == 0 && g.lda >= g.I, "float A rows must hold whole chunks of I");
        if (ak == kAFloatT) DLLM_REQUIRE(!seg && g.l0 == 0 && g.l1 % 4 == 0 && g.l1 >= 4 && g.lda >= g.l1,
                                         "transposed float A needs a plain reduction over whole 16-byte chunks");
        ps[k] = params_of(g);
    }
    DLLM_REQUIRE(max_tiles >= 1 && max_tiles < (int64_t{1} << 28), "row group too large for one launch");
    group->count = n;
    group->capacity = capacity;
    group->tile = tile;
    group->tiles = max_tiles;  // an upper bound: the kernel finds each workgroup's tile in the live table
    group->a_kind = ak;
    group->segmented = seg ? 1 : 0;
    // the fill keeps every XCD range within cap tiles: twice an even share leaves room for the equal-work cuts
    group->grid = 2 * static_cast<int64_t>(ceil_div(static_cast<size_t>(max_tiles), kXcdRanges)) * kXcdRanges;
    return kOk;
}

int launch_gemm_row_group_fill(const void* device_templ, void* device_table, const GemmGroup& group,
                               const int64_t* device_start, const GemmRowShift& shift, hipStream_t stream) {
    hipLaunchKernelGGL(gemm_row_group_fill_kernel, dim3(1), dim3(256), 0, stream,
                       static_cast<const GemmParams*>(device_templ), static_cast<GemmParams*>(device_table),
                       group.count, group.capacity, device_start, shift, group.tile, group.grid / kXcdRanges);
    return check_launch("gemm row group fill");
}

int launch_gemm_group(const GemmGroup& group, const void* device_table, hipStream_t stream) {
    if (group.tiles == 0) return kOk;
    const GemmParams* ps = static_cast<const GemmParams*>(device_table);
    // the tile table sits after the capacity the table was laid out for
    const int64_t* starts = reinterpret_cast<const int64_t*>(
        static_cast<const char*>(device_table) + round_up(sizeof(GemmParams) * static_cast<size_t>(group.capacity), 8));
    const GemmParams none{};
    const dim3 grid(static_cast<unsigned>(group.grid));
    DLLM_REQUIRE(group.grid < (int64_t{1} << 31), "matmul group too large for one launch");
    DLLM_REQUIRE(group.tile == 4 || (!group.segmented && (group.tile == 2 || group.tile == 1)),
                 "grouped matmul tiles are 128, or for plain groups 64 or 32, square");
#define DLLM_GROUP_LAUNCH(MODE, AK, T)                                                                            \
    hipLaunchKernelGGL((gemm_mfma_kernel<MODE, AK, true, T, T>), grid, dim3(256), 0, stream, none, group.tiles, \
                       int64_t{group.capacity}, int64_t{1}, ps, starts, group.count)
    if (group.segmented) {
        DLLM_GROUP_LAUNCH(kWindowsInSequence, kAFloatRows, 4);
    } else if (group.a_kind == kAFloatT) {
        if (group.tile == 4) DLLM_GROUP_LAUNCH(kPlain, kAFloatT, 4);
        else if (group.tile == 2) DLLM_GROUP_LAUNCH(kPlain, kAFloatT, 2);
        else DLLM_GROUP_LAUNCH(kPlain, kAFloatT, 1);
    } else {
        if (group.tile == 4) DLLM_GROUP_LAUNCH(kPlain, kAFloatRows, 4);
        else if (group.tile == 2) DLLM_GROUP_LAUNCH(kPlain, kAFloatRows, 2);
        else DLLM_GROUP_LAUNCH(kPlain, kAFloatRows, 1);
    }
#undef DLLM_GROUP_LAUNCH
    return check_launch("gemm group");
}

int launch_gemm(const GemmCall& g, hipStream_t stream) {
    DLLM_REQUIRE(g.I >= 0 && g.J >= 0, "negative matmul size");
    DLLM_REQUIRE(g.seg == nullptr || g.nseg >= 1, "segmented matmul needs at least one segment");
    DLLM_REQUIRE(g.seg != nullptr || g.seg_addrow == nullptr, "per-window addends need segments");
    DLLM_REQUIRE(g.seg_rowscale == nullptr || g.seg != nullptr, "per-row factors are for windowed weight gradients");
    DLLM_REQUIRE(g.seg_weight == nullptr || g.seg != nullptr, "per-window factors are for windowed weight gradients");
    if (g.a_kind != kADouble && g.a_scratch != nullptr && !mfma_shape(g)) {
        // Float A in a shape the matrix-core kernel cannot stage (a size or a row stride that is not a whole number
        // of 16-byte chunks): A is widened into the caller's double scratch ([l][i], rows padded to whole tiles) and
        // the VALU kernels run the same per-output chain over l ascending, so the bits are those of any other path.
        if (g.I == 0 || g.J == 0) return kOk;
        const int64_t ld = padded_rows(g.I), L = g.l1;
        DLLM_REQUIRE(L >= 0 && L * ld <= g.a_scratch_cap, "matmul scratch too small for the widened operand");
        GemmCall d = g;
        if (g.a_kind == kAFloatRows)
            DLLM_TRY(launch_to_double(g.Af, L, g.I, g.lda, g.a_scratch, ld, nullptr, 0, stream));
        else
            DLLM_TRY(launch_to_double(g.Af, g.I, L, g.lda, nullptr, 0, g.a_scratch, ld, stream));
        d.a_kind = kADouble;
        d.A = g.a_scratch;
        d.lda = ld;
        d.Af = nullptr;
        d.a_scratch = nullptr;
        return launch_gemm(d, stream);
    }
    const int ak = g.a_kind;
    DLLM_REQUIRE(ak == kADouble || ak == kAFloatRows || ak == kAFloatT, "unknown A operand kind");
    if (ak == kADouble) DLLM_REQUIRE(g.lda >= padded_rows(g.I), "the double operand must be padded to whole row tiles");
    if (g.I == 0 || g.J == 0) return kOk;
    GemmParams p = params_of(g);
    const bool vec = (g.J % 4 == 0) && (g.ldb % 4 == 0) && (reinterpret_cast<uintptr_t>(g.B) % 16 == 0);
    if (ak != kADouble) {
        // float A: 16-byte chunks of whole rows (and, transposed, a plain reduction over l in [0, l1))
        DLLM_REQUIRE(vec, "float A operands need B rows of whole 16-byte chunks");
        DLLM_REQUIRE(mfma_offsets_fit(g), "matmul operand rows too long for the matrix-core kernel's copy offsets");
        DLLM_REQUIRE(g.lda % 4 == 0 && reinterpret_cast<uintptr_t>(g.Af) % 16 == 0, "float A rows must be 16-byte aligned");
        if (ak == kAFloatRows) DLLM_REQUIRE(g.I % 4 == 0 && g.lda >= g.I, "float A rows must hold whole chunks of I");
        if (ak == kAFloatT)
            DLLM_REQUIRE(g.seg == nullptr && g.l0 == 0 && g.l1 % 4 == 0 && g.l1 >= 4 && g.lda >= g.l1,
                         "transposed float A needs a plain reduction over whole 16-byte chunks");
    }
    if (vec && (ak != kADouble || ((g.lda % 2 == 0) && (reinterpret_cast<uintptr_t>(g.A) % 16 == 0)))) {
        const bool mfma = ak != kADouble;
        int64_t gx = mfma ? ceil_div(g.J, MTile<4, 4>::J) : ceil_div(g.J, kTileJ);
        int64_t gy = mfma ? ceil_div(g.I, MTile<4, 4>::I) : ceil_div(g.I, kBlockI);
        int64_t gz = 1;
        // windows in parallel when the tile grid alone leaves most of the 256 CUs x 3 workgroups idle
        if (g.seg && g.nseg > 1 && g.seg_partial && gx * gy < kParallelWindowsBelow &&
            static_cast<int64_t>(g.nseg) * g.I * g.J <= g.seg_partial_cap) {
            p.partial = g.seg_partial;
            gz = g.nseg;
        }
        // matrix-core tiles: 128 x 128, or 64 x 64 / 32 x 32 when the larger tiles' grid leaves CUs idle (128 x 192
        // tiles, which fit a [rows x 1536] output in one round of the 512 workgroup slots, measured slower)
        int tile = 4;
        if (mfma) {
            while (tile > 1 && gx * gy * gz < kSmallTilesBelow) {
                tile /= 2;
                gx = ceil_div(g.J, 32 * tile);
                gy = ceil_div(g.I, 32 * tile);
            }
        }
        DLLM_REQUIRE(gx * gy * gz < (int64_t{1} << 31), "matmul grid too large for one launch");
        const dim3 grid(static_cast<unsigned>(gx * gy * gz));
#define DLLM_GEMM_LAUNCH(MODE, AK) \
    hipLaunchKernelGGL((gemm_lds_kernel<MODE, AK>), grid, dim3(256), 0, stream, p, gx, gy, gz, nullptr, nullptr, 0)
#define DLLM_GEMM_MFMA_T(MODE, AK, T)                                                                            \
    hipLaunchKernelGGL((gemm_mfma_kernel<MODE, AK, false, T, T>), grid, dim3(256), 0, stream, p, gx, gy, gz, nullptr, \
                       nullptr, 0)
#define DLLM_GEMM_MFMA(MODE, AK)                        \
    do {                                                \
        if (tile == 4) DLLM_GEMM_MFMA_T(MODE, AK, 4);   \
        else if (tile == 2) DLLM_GEMM_MFMA_T(MODE, AK, 2); \
        else DLLM_GEMM_MFMA_T(MODE, AK, 1);             \
    } while (0)
        if (ak == kAFloatT) {
            DLLM_GEMM_MFMA(kPlain, kAFloatT);
        } else if (ak == kAFloatRows) {
            if (p.partial) DLLM_GEMM_MFMA(kWindowsInParallel, kAFloatRows);
            else if (g.seg) DLLM_GEMM_MFMA(kWindowsInSequence, kAFloatRows);
            else DLLM_GEMM_MFMA(kPlain, kAFloatRows);
        } else {
            if (p.partial) DLLM_GEMM_LAUNCH(kWindowsInParallel, kADouble);
            else if (g.seg) DLLM_GEMM_LAUNCH(kWindowsInSequence, kADouble);
            else DLLM_GEMM_LAUNCH(kPlain, kADouble);
        }
#undef DLLM_GEMM_LAUNCH
#undef DLLM_GEMM_MFMA
#undef DLLM_GEMM_MFMA_T
        DLLM_TRY(check_launch("gemm"));
        if (p.partial) {
            const int64_t n = g.I * g.J;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 256), 8192));
            if (g.ldc == g.J && (g.I * g.J) % 4 == 0 && reinterpret_cast<uintptr_t>(g.C) % 16 == 0 &&
                reinterpret_cast<uintptr_t>(p.partial) % 16 == 0)
                hipLaunchKernelGGL(window_sum4_kernel, dim3(blocks), dim3(256), 0, stream,
                                   reinterpret_cast<const float4*>(p.partial), g.I * g.J / 4, g.nseg,
                                   reinterpret_cast<float4*>(g.C));
            else
                hipLaunchKernelGGL(window_sum_kernel, dim3(blocks), dim3(256), 0, stream, p.partial, g.I, g.J, g.nseg,
                                   g.C, g.ldc);
            return check_launch("gemm window sum");
        }
        return kOk;
    }
    DLLM_REQUIRE(ak == kADouble, "float A operands need the LDS matmul");
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

int64_t transpose_batch_tiles(const TransposeJob* jobs, int n, int64_t* tile_start) {
    int64_t tiles = 0;
    for (int k = 0; k < n; ++k) {
        tile_start[k] = tiles;
        tiles += static_cast<int64_t>(ceil_div(jobs[k].rows, 64) * ceil_div(jobs[k].cols, 64));
    }
    tile_start[n] = tiles;
    return tiles;
}

int launch_transpose_batch(const TransposeJob* device_jobs, const int64_t* device_tile_start, int n, int64_t tiles,
                           hipStream_t stream) {
    if (tiles == 0) return kOk;
    DLLM_REQUIRE(tiles < (int64_t{1} << 31), "too many transpose tiles for one launch");
    hipLaunchKernelGGL(transpose_batch_kernel, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, stream, device_jobs,
                       device_tile_start, n);
    return check_launch("transpose batch");
}

int launch_transpose_f32(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t stream) {
    if (rows == 0 || cols == 0) return kOk;
    dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
    DLLM_REQUIRE(grid.y <= 65535u, "too many rows for one transpose launch");
    hipLaunchKernelGGL(transpose_f32_kernel, grid, dim3(256), 0, stream, src, rows, cols, dst);
    return check_launch("transpose");
}

}  // namespace dllm_hip
