// Causal grouped-query attention of the training step as batched matmuls plus per-query-row chains
// (nn.hpp:535-615 forward, grad.hpp:206-301 backward), for every window and head of a step at once.
//
// Layout: scores are kept transposed, S^T[j][t] (key j, query t) per (window, head), so the columns a query owns are
// contiguous across queries: the softmax chains (first maximum, exponentials, their serial total; the backward's
// D = sum_j p_j dp_j) run one lane per query over keys ascending, with coalesced loads, and the matmuls find their
// wave-uniform operand rows contiguous.
//
//   forward   S^T = K Q^T * scale   (double, head_dim ascending, exact float products: fma)
//             E^T = exp(S^T - max_t), total_t serial, inv_t = 1 / total_t       (one lane per query)
//             out[t] = f32((sum_j E^T[j][t] v[j]) * inv_t)                         (keys ascending, multiply then add)
//   backward  P^T = E^T * inv_t;  dP^T = V dOut^T (double, exact products)
//             D_t = sum_j p dp (serial), dS^T = p (dp - D) scale                     (one lane per query)
//             dq[t] = f32(sum_j dS[t][j] k[j])                                       (keys ascending)
//             dk[j] = f32(sum over (t ascending, head of the group ascending) dS q), dv[j] likewise with p and dOut
// Each reduction runs exactly over the keys (or queries) the reference visits, in its order: the steps only some rows
// of a tile take run in separate per-output kernels before and after the tile's common steps, never fed zeros.
#include "attn_gemm.h"
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

struct Operand {
    const void* ptr;
    int64_t w_stride, seg_stride, head_stride;  // base = ptr + w*w_stride + seg[w]*seg_stride + (hz/head_div)*head_stride
    int64_t head_div;
    int64_t ld, ld_inner, group;  // row(l) = (l / group) * ld + (l % group) * ld_inner
};

template <typename T>
__device__ __forceinline__ const T* base_of(const Operand& o, int64_t w, int64_t seg_w, int64_t hz) {
    return static_cast<const T*>(o.ptr) + w * o.w_stride + seg_w * o.seg_stride + (hz / o.head_div) * o.head_stride;
}

struct AttnGemmParams {
    Operand A, B, C;
    const double* rowscale;  // per (z, row) multiplier before rounding (out = acc * inv); may be null
    int64_t rowscale_zstride;
    const int64_t* seg;
    int64_t heads;    // z = w * heads + hz
    int rows_kind;    // I = n_w (positions) if 0, head_dim if 1
    int cols_kind;    // J = n_w if 0, head_dim if 1
    int64_t head_dim;
    int64_t group;    // G for the key-row limits
    int mask;         // kMaskNone, kMaskQueryRows, kMaskKeyRows, kMaskTileCausal
    int64_t window;
    int64_t L;        // reduction length when unmasked (head_dim)
    double out_scale; // double outputs: value = acc * out_scale
    int64_t b_row_alloc;  // floats readable in each B row from column 0 (multiple of 4, >= J)
    double* partial;      // running sums between the edge and body kernels: [z][i][j]
    int64_t partial_zstride, partial_ld;
    int cols_per_lane;
    int tile_rows;        // 8 or 16 (the edge kernels rebuild the body kernel's tiles)
};

// The keys query t sees (causal, q_offset 0, optional window): [lo, hi).
__device__ __forceinline__ void query_span(int64_t t, int64_t window, int64_t* lo, int64_t* hi) {
    *hi = t + 1;
    *lo = window != 0 && t + 1 > window ? t + 1 - window : 0;
}

// The (t, head-in-group) rows that see key j, as l = t * G + hh: [lo, hi).
__device__ __forceinline__ void key_span(int64_t j, int64_t n, int64_t window, int64_t G, int64_t* lo, int64_t* hi) {
    *lo = j * G;
    const int64_t t_hi = window != 0 && j + window - 1 < n - 1 ? j + window - 1 : n - 1;
    *hi = (t_hi + 1) * G;
}

// 16 bytes global -> LDS at lds_row + 16 * lane (gfx950 direct-to-LDS load, M0 = LDS address). Inline assembly keeps
// the compiler's wait-count pass from stalling reads of the current stage on the next stage's copies; the kernel
// waits for its copies explicitly.
__device__ __forceinline__ void copy16_to_lds(const void* src, const void* lds_row) {
    typedef __attribute__((address_space(3))) const void* lds_address;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_address)lds_row));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

template <int kPending>
__device__ __forceinline__ void wait_copies() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPending) : "memory");
}

// A body tile: TI rows (8 or 16) x 64 CJ columns, one wave; a stage holds TI x (128 / TI) = 128 A values (1 KB, one
// copy) and 128 / TI rows of 64 CJ B values.
template <int CJ, int TI>
struct Tile {
    static constexpr int kSteps = 128 / TI;            // reduction steps per LDS stage
    static constexpr int kBCopies = kSteps * CJ / 4;   // 16-byte copies per lane for B
    static constexpr int kCopies = 1 + kBCopies;
    static constexpr int kBuffers = CJ == 4 ? 2 : CJ == 2 ? 3 : 4;  // stages in flight (LDS: 5-18 KB per workgroup)
    struct Stage {
        double a[kSteps][TI];
        float b[kSteps][64 * CJ];
    };
};

// acc[Q][c] = fma(A[l][i0 + Q], b[c], acc[Q][c]): lane L's `a` holds A[l][i0 + L % TI] and the DPP64 modifier
// row_newbcast:Q on the FMA hands lane Q of each 16-lane row to the whole row. s_nop 1: the two wait states a DPP
// source needs after a vector write (the compiler's hazard checks do not look inside the statement).
template <int CJ, int TI, int Q>
__device__ __forceinline__ void fma_bcast(double (&acc)[TI][CJ], double a, const double (&b)[CJ]) {
    if constexpr (CJ == 4)
        asm("s_nop 1\n\t"
            "v_fmac_f64_dpp %0, %4, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f64_dpp %1, %4, %6 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f64_dpp %2, %4, %7 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f64_dpp %3, %4, %8 row_newbcast:%9 row_mask:0xf bank_mask:0xf"
            : "+v"(acc[Q][0]), "+v"(acc[Q][1]), "+v"(acc[Q][2]), "+v"(acc[Q][3])
            : "v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "n"(Q));
    else if constexpr (CJ == 2)
        asm("s_nop 1\n\t"
            "v_fmac_f64_dpp %0, %2, %3 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f64_dpp %1, %2, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf"
            : "+v"(acc[Q][0]), "+v"(acc[Q][1])
            : "v"(a), "v"(b[0]), "v"(b[1]), "n"(Q));
    else
        asm("s_nop 1\n\t"
            "v_fmac_f64_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
            : "+v"(acc[Q][0])
            : "v"(a), "v"(b[0]), "n"(Q));
}

// A[l][i0 + Q + k] in every lane for k < 4 (lane Q + k of each 16-lane row, broadcast by DPP64 moves); four at a
// time so the products that follow are four independent chains.
template <int Q>
__device__ __forceinline__ void broadcast_rows4(double a, double (&r)[4]) {
    asm("s_nop 1\n\t"
        "v_mov_b64_dpp %0, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b64_dpp %1, %4 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b64_dpp %2, %4 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b64_dpp %3, %4 row_newbcast:%8 row_mask:0xf bank_mask:0xf"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a), "n"(Q), "n"(Q + 1), "n"(Q + 2), "n"(Q + 3));
}

// The reduction steps of tile rows i0 .. i0 + rows - 1 (rows past I behave like row I - 1 and are never stored)
// split in three ascending parts per row: a ragged head [lo(i), m0), a body [m0, m1) that every row of the tile
// takes, in whole LDS stages, and a ragged tail [m1, hi(i)). The body runs in the pipelined matmul kernel; the head
// before it and the tail after it run in one-thread-per-output kernels (attn_edge_kernel), the running double sum
// passed through `partial` - so each output is still one accumulation over its steps in the reference's order.
struct TileSplit {
    int64_t m0, m1;   // the body
    bool head, tail;  // some row has steps before m0 / after m1
};

__device__ __forceinline__ void row_span(const AttnGemmParams& p, int64_t r, int64_t n, int64_t* lo, int64_t* hi) {
    if (p.mask == kMaskQueryRows) {
        query_span(r, p.window, lo, hi);
    } else if (p.mask == kMaskKeyRows) {
        key_span(r, n, p.window, p.group, lo, hi);
    } else {
        *lo = 0;
        *hi = p.L;
    }
}

__device__ __forceinline__ TileSplit tile_split(const AttnGemmParams& p, int64_t i0, int64_t rows, int64_t steps,
                                                int64_t I, int64_t n) {
    // the spans' ends are non-decreasing in the row, so the tile's first and last rows bound them
    const int64_t r_last = i0 + rows - 1 < I ? i0 + rows - 1 : I - 1;
    int64_t lo_f, hi_f, lo_l, hi_l;
    row_span(p, i0, n, &lo_f, &hi_f);
    row_span(p, r_last, n, &lo_l, &hi_l);
    TileSplit t;
    if (lo_l < hi_f) {  // steps every row takes: [lo_l, hi_f)
        t.m0 = lo_l;
        t.m1 = lo_l + (hi_f - lo_l) / steps * steps;
    } else {
        t.m0 = t.m1 = lo_l;
    }
    t.head = lo_f < t.m0;
    t.tail = hi_l > t.m1;
    return t;
}

// S^T / dP^T tiles (rows keys j, columns queries t) none of whose queries sees any of their keys are skipped.
__device__ __forceinline__ bool tile_unseen(const AttnGemmParams& p, int64_t i0, int64_t rows, int64_t jw0,
                                            int64_t cols) {
    if (p.mask != kMaskTileCausal) return false;
    if (i0 > jw0 + cols - 1) return true;
    return p.window != 0 && i0 + rows - 1 + p.window - 1 < jw0;
}

template <int CJ>
struct RowOperands {
    double a;
    float b[CJ];
};

template <int CJ, int TI>
__device__ __forceinline__ RowOperands<CJ> read_row(const typename Tile<CJ, TI>::Stage& st, int k, int lane) {
    RowOperands<CJ> r;
    r.a = st.a[k][lane & (TI - 1)];
    if constexpr (CJ == 4) {
        const float4 v = *reinterpret_cast<const float4*>(&st.b[k][lane * 4]);
        r.b[0] = v.x; r.b[1] = v.y; r.b[2] = v.z; r.b[3] = v.w;
    } else if constexpr (CJ == 2) {
        const float2 v = *reinterpret_cast<const float2*>(&st.b[k][lane * 2]);
        r.b[0] = v.x; r.b[1] = v.y;
    } else {
        r.b[0] = st.b[k][lane];
    }
    return r;
}

// One step for every row of the tile: exact products by fused multiply-add, the others as a rounded product then a
// rounded sum (four rows at a time).
template <int CJ, int TI, bool kExact, int Q>
__device__ __forceinline__ void step_rows(double (&acc)[TI][CJ], double a, const double (&b)[CJ]) {
    if constexpr (Q < TI) {
        if constexpr (kExact) {
            fma_bcast<CJ, TI, Q>(acc, a, b);
            step_rows<CJ, TI, kExact, Q + 1>(acc, a, b);
        } else {
            double aq[4];
            broadcast_rows4<Q>(a, aq);
            double prod[4][CJ];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int c = 0; c < CJ; ++c) prod[k][c] = aq[k] * b[c];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int c = 0; c < CJ; ++c) acc[Q + k][c] = acc[Q + k][c] + prod[k][c];
            step_rows<CJ, TI, kExact, Q + 4>(acc, a, b);
        }
    }
}

// Copies of the stage holding steps l .. l + kSteps - 1.
template <int CJ, int TI>
__device__ __forceinline__ void issue_stage(typename Tile<CJ, TI>::Stage& st, const double* a_base, int64_t lda,
                                            const float* b_base, const Operand& bo, int64_t b_col, int64_t l,
                                            int lane) {
    using T = Tile<CJ, TI>;
    // A: kSteps rows x TI doubles (TI / 2 lanes per row), lane L -> row L / (TI / 2), doubles 2 (L % (TI / 2)) .. + 1
    copy16_to_lds(a_base + (l + lane / (TI / 2)) * lda + (lane % (TI / 2)) * 2, &st.a[0][0]);
    // B: kSteps rows x 64 CJ floats, 16 CJ lanes per row; b_col is this lane's chunk (see run_tile). Row offsets
    // stepped from one (uniform, scalar) division
    int64_t off[T::kSteps];
    {
        int64_t t = l / bo.group, hh = l % bo.group;
#pragma unroll
        for (int r = 0; r < T::kSteps; ++r) {
            off[r] = t * bo.ld + hh * bo.ld_inner;
            if (++hh == bo.group) {
                hh = 0;
                ++t;
            }
        }
    }
    constexpr int kLanesPerRow = 16 * CJ;
    constexpr int kRowsPerCopy = 64 / kLanesPerRow;
    const int sub = lane / kLanesPerRow;
#pragma unroll
    for (int t = 0; t < T::kBCopies; ++t) {
        int64_t row = off[t * kRowsPerCopy];
#pragma unroll
        for (int k = 1; k < kRowsPerCopy; ++k)
            if (sub == k) row = off[t * kRowsPerCopy + k];
        copy16_to_lds(b_base + row + b_col, &st.b[t * kRowsPerCopy][0]);
    }
}

// The steps of a stage, unrolled; the next step's operands are read from LDS while this step's products run.
template <int CJ, int TI, bool kExact>
__device__ __forceinline__ void stage_steps(const typename Tile<CJ, TI>::Stage& st, int lane, double (&acc)[TI][CJ]) {
    using T = Tile<CJ, TI>;
    RowOperands<CJ> cur = read_row<CJ, TI>(st, 0, lane);
#pragma unroll
    for (int k = 0; k < T::kSteps; ++k) {
        RowOperands<CJ> next = cur;
        if (k + 1 < T::kSteps) next = read_row<CJ, TI>(st, k + 1, lane);
        double bd[CJ];
#pragma unroll
        for (int c = 0; c < CJ; ++c) bd[c] = cur.b[c];
        step_rows<CJ, TI, kExact, 0>(acc, cur.a, bd);
        cur = next;
    }
}

// Where a running sum waits between kernels: the double output itself (finished in place by the tail kernel), or
// the float outputs' scratch [z][i][j].
template <bool kOutDouble>
__device__ __forceinline__ double* partial_base(const AttnGemmParams& p, int64_t w, int64_t seg_w, int64_t hz,
                                                int64_t z, int64_t* ld) {
    if (kOutDouble) {
        *ld = p.C.ld;
        return const_cast<double*>(base_of<double>(p.C, w, seg_w, hz));
    }
    *ld = p.partial_ld;
    return p.partial + z * p.partial_zstride;
}

template <bool kOutDouble>
__device__ __forceinline__ void store_output(const AttnGemmParams& p, int64_t w, int64_t seg_w, int64_t hz, int64_t z,
                                             int64_t i, int64_t j, double v) {
    if (kOutDouble) {
        double* C = const_cast<double*>(base_of<double>(p.C, w, seg_w, hz));
        C[i * p.C.ld + j] = v * p.out_scale;
    } else {
        float* C = const_cast<float*>(base_of<float>(p.C, w, seg_w, hz));
        if (p.rowscale) v = v * p.rowscale[z * p.rowscale_zstride + i];
        C[i * p.C.ld + j] = static_cast<float>(v);
    }
}

// The body of one TI-row x 64 CJ-column tile of (window, head) z: acc[q][c] (+)= sum over l in [m0, m1), ascending,
// of A_z[l][i0 + q] * B_z[l][jw0 + lane CJ + c]; operands staged through LDS in a ring of stages filled by gfx950's
// direct-to-LDS loads.
template <int CJ, int TI, bool kExact, bool kOutDouble>
__device__ __forceinline__ void run_tile(const AttnGemmParams& p, typename Tile<CJ, TI>::Stage* st, int lane,
                                         int64_t z, int64_t w, int64_t hz, int64_t seg_w, int64_t n, int64_t I,
                                         int64_t J, int64_t i0, int64_t jw0) {
    using T = Tile<CJ, TI>;
    if (i0 >= I || jw0 >= J || tile_unseen(p, i0, TI, jw0, 64 * CJ)) return;  // workgroup-uniform
    const TileSplit ts = tile_split(p, i0, TI, T::kSteps, I, n);
    const double* A = base_of<double>(p.A, w, seg_w, hz) + i0;
    const float* B = base_of<float>(p.B, w, seg_w, hz);
    // this lane's 16-byte B chunk in each row: columns jw0 + 4 (lane % 16 CJ) .. + 3; chunks past the readable row
    // (b_row_alloc, a multiple of 4 that is >= J) read its last chunk instead, and their columns are never stored
    const int64_t chunk = jw0 + 4 * (lane % (16 * CJ));
    const int64_t b_col = chunk + 4 <= p.b_row_alloc ? chunk : p.b_row_alloc - 4;
    int64_t part_ld;
    double* part = partial_base<kOutDouble>(p, w, seg_w, hz, z, &part_ld);
    double acc[TI][CJ];
#pragma unroll
    for (int q = 0; q < TI; ++q)
#pragma unroll
        for (int c = 0; c < CJ; ++c) {
            const int64_t i = i0 + q, j = jw0 + lane * CJ + c;
            acc[q][c] = ts.head && i < I && j < J ? part[i * part_ld + j] : 0.0;
        }
    // consume the loaded sums here, so the wait for them is placed before the copy pipeline rather than inside it
    // (a vector-memory wait there would also drain the stage copies in flight)
#pragma unroll
    for (int q = 0; q < TI; ++q)
#pragma unroll
        for (int c = 0; c < CJ; ++c) asm volatile("" ::"v"(acc[q][c]));
    const int64_t stages = (ts.m1 - ts.m0) / T::kSteps;
    // a ring of kBuffers stages: stage s + kBuffers - 1 is requested before stage s is computed
    for (int64_t s0 = 0; s0 < T::kBuffers - 1 && s0 < stages; ++s0)
        issue_stage<CJ, TI>(st[s0], A, p.A.ld, B, p.B, b_col, ts.m0 + s0 * T::kSteps, lane);
    for (int64_t sidx = 0; sidx < stages; ++sidx) {
        const int64_t ahead = sidx + T::kBuffers - 1;
        if (ahead < stages)
            issue_stage<CJ, TI>(st[ahead % T::kBuffers], A, p.A.ld, B, p.B, b_col, ts.m0 + ahead * T::kSteps, lane);
        // stages issued after this one: min(kBuffers - 1, stages - 1 - sidx)
        const int64_t later = stages - 1 - sidx < T::kBuffers - 1 ? stages - 1 - sidx : T::kBuffers - 1;
        if (later >= 3)
            wait_copies<3 * T::kCopies>();
        else if (later == 2)
            wait_copies<2 * T::kCopies>();
        else if (later == 1)
            wait_copies<T::kCopies>();
        else
            wait_copies<0>();
        stage_steps<CJ, TI, kExact>(st[sidx % T::kBuffers], lane, acc);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this stage's reads are done before it is refilled
    }
#pragma unroll
    for (int q = 0; q < TI; ++q) {
        const int64_t i = i0 + q;
        if (i >= I) break;
#pragma unroll
        for (int c = 0; c < CJ; ++c) {
            const int64_t j = jw0 + lane * CJ + c;
            if (j >= J) continue;
            if (ts.tail)
                part[i * part_ld + j] = acc[q][c];
            else
                store_output<kOutDouble>(p, w, seg_w, hz, z, i, j, acc[q][c]);
        }
    }
}

// One workgroup (one wave) runs row tiles y and tiles - 1 - y of one (z, column block): the tiles' serial
// reductions grow (or shrink) with the row, so every workgroup gets about the same total work.
template <int CJ, int TI, bool kExact, bool kOutDouble>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(CJ == 4 ? 3 : 4))) void attn_gemm_kernel(
    AttnGemmParams p) {
    using T = Tile<CJ, TI>;
    __shared__ typename T::Stage st[T::kBuffers];
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t z = blockIdx.z;
    const int64_t w = z / p.heads, hz = z % p.heads;
    const int64_t seg_w = p.seg[w], n = p.seg[w + 1] - seg_w;
    const int64_t I = p.rows_kind == 0 ? n : p.head_dim;
    const int64_t J = p.cols_kind == 0 ? n : p.head_dim;
    const int64_t tiles = (I + TI - 1) / TI;
    const int64_t y = blockIdx.y, y2 = tiles - 1 - y;
    const int64_t jw0 = static_cast<int64_t>(blockIdx.x) * 64 * CJ;
    if (y > y2) return;
    run_tile<CJ, TI, kExact, kOutDouble>(p, st, lane, z, w, hz, seg_w, n, I, J, y * TI, jw0);
    if (y2 != y) run_tile<CJ, TI, kExact, kOutDouble>(p, st, lane, z, w, hz, seg_w, n, I, J, y2 * TI, jw0);
}

// The ragged head (kHead) or tail of every output: one thread per (z, i, j), continuing the running sum in `partial`
// over its row's steps outside the tile body, then (tail) rounding and storing the output.
template <bool kHead, bool kExact, bool kOutDouble>
__global__ __launch_bounds__(256) void attn_edge_kernel(AttnGemmParams p, int64_t max_i, int64_t max_j) {
    const int64_t z = blockIdx.z;
    const int64_t w = z / p.heads, hz = z % p.heads;
    const int64_t seg_w = p.seg[w], n = p.seg[w + 1] - seg_w;
    const int64_t I = p.rows_kind == 0 ? n : p.head_dim;
    const int64_t J = p.cols_kind == 0 ? n : p.head_dim;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + (threadIdx.x & 63);
    const int64_t i = static_cast<int64_t>(blockIdx.y) * 4 + (threadIdx.x >> 6);
    if (i >= I || j >= J || i >= max_i || j >= max_j) return;
    const int64_t rows = p.tile_rows, cols = 64 * p.cols_per_lane;
    const int64_t i0 = i / rows * rows;
    if (tile_unseen(p, i0, rows, j / cols * cols, cols)) return;  // the body kernel's tiles
    const TileSplit ts = tile_split(p, i0, rows, 128 / rows, I, n);
    if (kHead ? !ts.head : !ts.tail) return;
    int64_t lo, hi;
    row_span(p, i, n, &lo, &hi);
    int64_t from, to;
    if (kHead) {
        from = lo;
        to = hi < ts.m0 ? hi : ts.m0;
    } else {
        from = lo > ts.m1 ? lo : ts.m1;
        to = hi;
    }
    int64_t part_ld;
    double* part = partial_base<kOutDouble>(p, w, seg_w, hz, z, &part_ld) + i * part_ld + j;
    double acc = kHead ? 0.0 : *part;
    const double* A = base_of<double>(p.A, w, seg_w, hz) + i;
    const float* B = base_of<float>(p.B, w, seg_w, hz) + j;
    for (int64_t l = from; l < to; ++l) {
        const double a = A[l * p.A.ld];
        const double b = static_cast<double>(B[(l / p.B.group) * p.B.ld + (l % p.B.group) * p.B.ld_inner]);
        acc = kExact ? __builtin_fma(a, b, acc) : acc + a * b;
    }
    if (kHead)
        *part = acc;
    else
        store_output<kOutDouble>(p, w, seg_w, hz, z, i, j, acc);
}

// The forward softmax of every query (nn.hpp:541-561) in three passes over S^T (keys j, queries t; one lane per query
// where the reference's order matters, every element in parallel where it does not):
//   softmax_max_kernel    mx_t = first maximum over the visible keys, ascending (strictly greater replaces)
//   softmax_exp_kernel    e = exp(s - mx_t) written over S^T (each element independent)
//   softmax_total_kernel  total_t = sum of e over the visible keys ascending, inv_t = 1 / total_t
// The lanes' loads are issued 8 keys ahead of their serial use.
constexpr int kChainUnroll = 8;

__global__ __launch_bounds__(64) void softmax_max_kernel(const double* __restrict__ st, int64_t ld, int64_t zstride,
                                                         const int64_t* __restrict__ seg, int64_t heads,
                                                         int64_t window, double* __restrict__ mx_out,
                                                         int64_t mx_zstride) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    const double* s = st + z * zstride + t;
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    double mx = s[lo * ld];
    int64_t j = lo + 1;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = s[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k)
            if (v[k] > mx) mx = v[k];
    }
    for (; j < hi; ++j) {
        const double v = s[j * ld];
        if (v > mx) mx = v;
    }
    mx_out[z * mx_zstride + t] = mx;
}

// 256 queries x 8 keys per workgroup.
__global__ __launch_bounds__(256) void softmax_exp_kernel(double* __restrict__ st, int64_t ld, int64_t zstride,
                                                          const int64_t* __restrict__ seg, int64_t heads,
                                                          int64_t window, const double* __restrict__ mx,
                                                          int64_t mx_zstride) {
    const int64_t z = blockIdx.z;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t j0 = static_cast<int64_t>(blockIdx.y) * 8;
    if (t >= n || j0 > t) return;
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    const double m = mx[z * mx_zstride + t];
    double* s = st + z * zstride + t;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int64_t j = j0 + k;
        if (j >= lo && j < hi) s[j * ld] = dexp(s[j * ld] - m);
    }
}

__global__ __launch_bounds__(64) void softmax_total_kernel(const double* __restrict__ st, int64_t ld, int64_t zstride,
                                                           const int64_t* __restrict__ seg, int64_t heads,
                                                           int64_t window, double* __restrict__ inv,
                                                           int64_t inv_zstride) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    const double* s = st + z * zstride + t;
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    double total = 0.0;
    int64_t j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double v[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) v[k] = s[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) total += v[k];
    }
    for (; j < hi; ++j) total += s[j * ld];
    inv[z * inv_zstride + t] = 1.0 / total;
}

// The backward chains per query (grad.hpp:262-278) in two passes:
//   dsoftmax_dot_kernel    D_t = sum over visible keys ascending of (e inv_t) dp (one lane per query)
//   dsoftmax_apply_kernel  p = e inv_t over E^T and ds = (p (dp - D_t)) scale over dP^T (each element independent)
__global__ __launch_bounds__(64) void dsoftmax_dot_kernel(const double* __restrict__ et, const double* __restrict__ dpt,
                                                          int64_t ld, int64_t zstride,
                                                          const int64_t* __restrict__ seg, int64_t heads,
                                                          int64_t window, const double* __restrict__ inv,
                                                          int64_t inv_zstride, double* __restrict__ dvec) {
    const int64_t z = blockIdx.y;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (t >= n) return;
    const double* e = et + z * zstride + t;
    const double* d = dpt + z * zstride + t;
    const double iv = inv[z * inv_zstride + t];
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    double weighted = 0.0;
    int64_t j = lo;
    for (; j + kChainUnroll <= hi; j += kChainUnroll) {
        double term[kChainUnroll];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) term[k] = (e[(j + k) * ld] * iv) * d[(j + k) * ld];
#pragma unroll
        for (int k = 0; k < kChainUnroll; ++k) weighted += term[k];
    }
    for (; j < hi; ++j) weighted += (e[j * ld] * iv) * d[j * ld];
    dvec[z * inv_zstride + t] = weighted;
}

__global__ __launch_bounds__(256) void dsoftmax_apply_kernel(double* __restrict__ et, double* __restrict__ dpt,
                                                             int64_t ld, int64_t zstride,
                                                             const int64_t* __restrict__ seg, int64_t heads,
                                                             int64_t window, const double* __restrict__ inv,
                                                             int64_t inv_zstride, const double* __restrict__ dvec,
                                                             double scale) {
    const int64_t z = blockIdx.z;
    const int64_t w = z / heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t j0 = static_cast<int64_t>(blockIdx.y) * 8;
    if (t >= n || j0 > t) return;
    int64_t lo, hi;
    query_span(t, window, &lo, &hi);
    const double iv = inv[z * inv_zstride + t];
    const double D = dvec[z * inv_zstride + t];
    double* e = et + z * zstride + t;
    double* d = dpt + z * zstride + t;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int64_t j = j0 + k;
        if (j >= lo && j < hi) {
            const double p = e[j * ld] * iv;
            e[j * ld] = p;
            d[j * ld] = p * (d[j * ld] - D) * scale;
        }
    }
}

// dst[w][g][(t * G + hh)][j] = src[w][g * G + hh][j][t] (doubles): the key-row operand layout of dk / dv.
__global__ __launch_bounds__(256) void regroup_kernel(const double* __restrict__ src, int64_t ld, int64_t zstride,
                                                      double* __restrict__ dst, int64_t dst_ld, int64_t dst_zstride,
                                                      const int64_t* __restrict__ seg, int64_t heads, int64_t group) {
    __shared__ double tile[64][65];
    const int64_t z = blockIdx.z;  // (w, h)
    const int64_t w = z / heads, h = z % heads;
    const int64_t g = h / group, hh = h % group;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t j0 = static_cast<int64_t>(blockIdx.y) * 64, t0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (j0 >= n || t0 >= n) return;
    const double* s = src + z * zstride;
    double* d = dst + (w * (heads / group) + g) * dst_zstride;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t j = j0 + k, t = t0 + tx;
        tile[k][tx] = (j < n && t < n) ? s[j * ld + t] : 0.0;
    }
    __syncthreads();
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, j = j0 + tx;
        if (t < n && j < n) d[(t * group + hh) * dst_ld + j] = tile[tx][k];
    }
}

// Per (window, head): dst[i][t] = src[(seg[w] + t) * row_stride + head * head_dim + i], as double or float.
template <typename T>
__global__ __launch_bounds__(256) void heads_transpose_kernel(const float* __restrict__ src, int64_t row_stride,
                                                              int64_t head_dim, T* __restrict__ dst, int64_t ld,
                                                              int64_t zstride, const int64_t* __restrict__ seg,
                                                              int64_t heads) {
    __shared__ float tile[64][65];
    const int64_t z = blockIdx.z;
    const int64_t w = z / heads, h = z % heads;
    const int64_t n = seg[w + 1] - seg[w];
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64, i0 = static_cast<int64_t>(blockIdx.y) * 64;
    if (t0 >= n || i0 >= head_dim) return;
    const float* s = src + seg[w] * row_stride + h * head_dim;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int k = ty; k < 64; k += 4) {
        const int64_t t = t0 + k, i = i0 + tx;
        tile[k][tx] = (t < n && i < head_dim) ? s[t * row_stride + i] : 0.0f;
    }
    __syncthreads();
    T* d = dst + z * zstride;
    for (int k = ty; k < 64; k += 4) {
        const int64_t i = i0 + k, t = t0 + tx;
        if (i < head_dim && t < n) d[i * ld + t] = static_cast<T>(tile[tx][k]);
    }
}

}  // namespace

int launch_attn_gemm(const AttnGemmCall& c, hipStream_t stream) {
    AttnGemmParams p;
    auto op = [](const AttnOperand& o) {
        return Operand{o.ptr, o.w_stride, o.seg_stride, o.head_stride, o.head_div > 0 ? o.head_div : 1, o.ld,
                       o.ld_inner, o.group > 0 ? o.group : 1};
    };
    p.A = op(c.A);
    p.B = op(c.B);
    p.C = op(c.C);
    p.rowscale = c.rowscale;
    p.rowscale_zstride = c.rowscale_zstride;
    p.seg = c.seg;
    p.heads = c.heads;
    p.rows_kind = c.rows_kind;
    p.cols_kind = c.cols_kind;
    p.head_dim = c.head_dim;
    p.group = c.group > 0 ? c.group : 1;
    p.mask = c.mask;
    p.window = c.window;
    p.L = c.L;
    p.out_scale = c.out_scale;
    const int64_t I = c.rows_kind == 0 ? c.max_len : c.head_dim;
    const int64_t J = c.cols_kind == 0 ? c.max_len : c.head_dim;
    const int64_t Z = c.windows * c.heads;
    p.b_row_alloc = c.b_row_alloc > 0 ? c.b_row_alloc : J;
    p.partial = c.scratch;
    p.partial_ld = J;
    p.partial_zstride = I * J;
    p.cols_per_lane = c.cols_per_lane;
    p.tile_rows = c.tile_rows;
    const int cj = c.cols_per_lane, ti = c.tile_rows;
    DLLM_REQUIRE((ti == 16 && (cj == 1 || cj == 2 || cj == 4)) || (ti == 8 && cj == 1),
                 "attention tiles are 16 rows x 64, 128 or 256 columns, or 8 rows x 64 columns");
    DLLM_REQUIRE(p.b_row_alloc % 4 == 0 && p.b_row_alloc >= J, "attention operand rows must hold whole 16-byte chunks");
    DLLM_REQUIRE(c.A.ld % 2 == 0 && c.A.ld >= static_cast<int64_t>(round_up(static_cast<size_t>(I), 16)),
                 "attention double operand rows must be padded to whole 16-row tiles");
    DLLM_REQUIRE(c.out_double || (c.scratch != nullptr && c.scratch_doubles >= Z * I * J),
                 "attention matmul scratch too small");
    if (I == 0 || J == 0 || Z == 0) return kOk;
    const dim3 body(static_cast<unsigned>(ceil_div(J, 64 * cj)), static_cast<unsigned>(ceil_div(ceil_div(I, ti), 2)),
                    static_cast<unsigned>(Z));
    const dim3 edge(static_cast<unsigned>(ceil_div(J, 64)), static_cast<unsigned>(ceil_div(I, 4)),
                    static_cast<unsigned>(Z));
    const bool heads_possible = c.mask == kMaskKeyRows || (c.mask == kMaskQueryRows && c.window != 0);
    const bool tails_possible = c.mask == kMaskQueryRows || c.mask == kMaskKeyRows || c.L % (128 / ti) != 0;
    const bool ex = c.exact_products, od = c.out_double;
#define DLLM_ATTN_EDGE(HEAD, EXACT, OUTD) \
    hipLaunchKernelGGL((attn_edge_kernel<HEAD, EXACT, OUTD>), edge, dim3(256), 0, stream, p, I, J)
#define DLLM_ATTN_EDGES(HEAD)                            \
    do {                                                \
        if (ex && od) DLLM_ATTN_EDGE(HEAD, true, true); \
        else if (ex) DLLM_ATTN_EDGE(HEAD, true, false); \
        else if (od) DLLM_ATTN_EDGE(HEAD, false, true); \
        else DLLM_ATTN_EDGE(HEAD, false, false);        \
    } while (0)
#define DLLM_ATTN_BODY(CJ, TI, EXACT, OUTD) \
    hipLaunchKernelGGL((attn_gemm_kernel<CJ, TI, EXACT, OUTD>), body, dim3(64), 0, stream, p)
#define DLLM_ATTN_BODIES(CJ, TI)                            \
    do {                                                   \
        if (ex && od) DLLM_ATTN_BODY(CJ, TI, true, true);  \
        else if (ex) DLLM_ATTN_BODY(CJ, TI, true, false);  \
        else if (od) DLLM_ATTN_BODY(CJ, TI, false, true);  \
        else DLLM_ATTN_BODY(CJ, TI, false, false);         \
    } while (0)
    if (heads_possible) DLLM_ATTN_EDGES(true);
    if (ti == 8) DLLM_ATTN_BODIES(1, 8);
    else if (cj == 4) DLLM_ATTN_BODIES(4, 16);
    else if (cj == 2) DLLM_ATTN_BODIES(2, 16);
    else DLLM_ATTN_BODIES(1, 16);
    if (tails_possible) DLLM_ATTN_EDGES(false);
#undef DLLM_ATTN_BODIES
#undef DLLM_ATTN_BODY
#undef DLLM_ATTN_EDGES
#undef DLLM_ATTN_EDGE
    return check_launch("attention matmul");
}

int launch_softmax_rows(double* st, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                        int64_t max_len, int64_t window, double* inv, int64_t inv_zstride, hipStream_t stream) {
    if (max_len == 0 || windows * heads == 0) return kOk;
    const dim3 lanes(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    const dim3 elems(static_cast<unsigned>(ceil_div(max_len, 256)), static_cast<unsigned>(ceil_div(max_len, 8)),
                     static_cast<unsigned>(windows * heads));
    // the maxima wait in `inv` until the totals replace them
    hipLaunchKernelGGL(softmax_max_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                       inv_zstride);
    hipLaunchKernelGGL(softmax_exp_kernel, elems, dim3(256), 0, stream, st, ld, zstride, seg, heads, window, inv,
                       inv_zstride);
    hipLaunchKernelGGL(softmax_total_kernel, lanes, dim3(64), 0, stream, st, ld, zstride, seg, heads, window, inv,
                       inv_zstride);
    return check_launch("attention softmax");
}

int launch_dsoftmax_rows(double* et, double* dpt, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows,
                         int64_t heads, int64_t max_len, int64_t window, const double* inv, int64_t inv_zstride,
                         double scale, double* dvec, hipStream_t stream) {
    if (max_len == 0 || windows * heads == 0) return kOk;
    const dim3 lanes(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(windows * heads));
    const dim3 elems(static_cast<unsigned>(ceil_div(max_len, 256)), static_cast<unsigned>(ceil_div(max_len, 8)),
                     static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(dsoftmax_dot_kernel, lanes, dim3(64), 0, stream, et, dpt, ld, zstride, seg, heads, window, inv,
                       inv_zstride, dvec);
    hipLaunchKernelGGL(dsoftmax_apply_kernel, elems, dim3(256), 0, stream, et, dpt, ld, zstride, seg, heads, window,
                       inv, inv_zstride, dvec, scale);
    return check_launch("attention softmax backward");
}

int launch_regroup(const double* src, int64_t ld, int64_t zstride, double* dst, int64_t dst_ld, int64_t dst_zstride,
                   const int64_t* seg, int64_t windows, int64_t heads, int64_t group, int64_t max_len,
                   hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(max_len, 64)),
              static_cast<unsigned>(windows * heads));
    hipLaunchKernelGGL(regroup_kernel, grid, dim3(256), 0, stream, src, ld, zstride, dst, dst_ld, dst_zstride, seg,
                       heads, group);
    return check_launch("attention regroup");
}

int launch_heads_transpose(const float* src, int64_t row_stride, int64_t head_dim, void* dst, bool to_double,
                           int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                           int64_t max_len, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_len, 64)), static_cast<unsigned>(ceil_div(head_dim, 64)),
              static_cast<unsigned>(windows * heads));
    if (to_double)
        hipLaunchKernelGGL(heads_transpose_kernel<double>, grid, dim3(256), 0, stream, src, row_stride, head_dim,
                           static_cast<double*>(dst), ld, zstride, seg, heads);
    else
        hipLaunchKernelGGL(heads_transpose_kernel<float>, grid, dim3(256), 0, stream, src, row_stride, head_dim,
                           static_cast<float*>(dst), ld, zstride, seg, heads);
    return check_launch("heads transpose");
}

}  // namespace dllm_hip
