// The attention matmuls of the training step (attn_step.h) as 64-row tiles through a double-buffered LDS pipeline,
// one workgroup of four waves per tile, every (window, head) of the step in one launch.
//
// Each output is C[i][j] = sum over l in row i's span, ascending, of A[l][i] * B[l][j] (then times a row scale or a
// constant), accumulated in double and rounded once:
//   scores      S^T[key][query] = sum_d K[key][d] Q[query][d]        exact products: matrix cores (attn_mfma_kernel)
//   dP^T        dP^T[key][query] = sum_d V[key][d] dOut[query][d]     (as above)
//   out, dq     row t (query): sum over the keys t sees of E^T / dS^T times V / K    A double: multiply, then add
//   dk, dv      row j (key): sum over (query t, head of the group) that see j of dS / P times Q / dOut  (as above)
// The products with a double factor are not exact, so they are a rounded multiply and a rounded add, as the
// reference computes them (grad.hpp:262-301, nn.hpp:535-569); attn_tile_kernel runs them on the vector ALU.
//
// (Measured alternatives: a ring of three LDS stages, two in flight, for the small grids of T = 256: 14% slower.
// Waves owning 8 rows by every column, the rows' A values scalar-loaded into SGPRs as
// multiply operands and B loaded per lane, no LDS: 106 against 63 ms per step at T = 1024, the scalar loads' latency
// exposed every few steps with only 64 SGPRs of them in flight.)
// attn_tile_kernel mapping: a wave owns 16 consecutive rows by 64 CJ columns; each lane holds a 4-row x 4 CJ-column
// register tile, so the LDS bytes read per multiply-add are few (the vector ALU, not the LDS, sets the pace). A stage
// is 16 consecutive l: the workgroup's A (16 l x 64 rows) is copied global -> LDS with gfx950's direct-to-LDS loads
// and B (16 l x 64 CJ columns) loaded into registers while the previous stage is computed, then widened to double
// as it is written to LDS.
// Causal rows have ragged spans: stages inside every row's span of the wave run unpredicated; at the ragged ends
// each (row, l) is taken only when l lies in that row's span (a wave-uniform test), so every row adds exactly its
// own steps, in order, and nothing else. Tiles are dispatched longest reduction first.
#include "attn_step.h"
#include "common.h"
#include "lds_copy.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

constexpr int kChunk = 16;  // reduction steps per stage
constexpr int kTileRows = 64;

struct Op {
    const void* ptr;
    int64_t w_stride, seg_stride, head_stride, head_div;
    int64_t ld, ld_inner, group;  // row(l) = (l / group) * ld + (l % group) * ld_inner
};

template <typename T>
__device__ __forceinline__ const T* op_base(const Op& o, int64_t w, int64_t seg_w, int64_t hz) {
    return static_cast<const T*>(o.ptr) + w * o.w_stride + seg_w * o.seg_stride + (hz / o.head_div) * o.head_stride;
}

// A wave-uniform 64-bit value the compiler cannot prove uniform (loaded through a pointer), kept in scalar registers.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint64_t u = static_cast<uint64_t>(v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u & 0xffffffffu)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32)));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

struct OperandSet {
    Op A, B, C;
};

struct TileParams {
    OperandSet set[2];         // one launch may run two matmuls of the same shape (dk and dv)
    int sets;
    const double* rowscale;    // float outputs: value * rowscale[z][i] before rounding; may be null
    int64_t rowscale_zstride;
    double out_scale;          // double outputs: value * out_scale
    double* tile_max;          // scores: per 64-key tile and query, the largest visible score (may be null)
    int64_t tile_max_zstride, tile_max_ld;
    const int64_t* seg;
    int64_t heads, Z;          // z = w * heads + hz in [0, Z)
    int rows_kind, cols_kind;  // 0: window positions, 1: head_dim
    int64_t head_dim, group, window, L;
    int mask;
    int64_t b_row_alloc;  // floats readable in each B row from column 0 (multiple of 4, >= J)
    int64_t a_row_alloc;  // float A: floats readable in each A row (multiple of 4)
    int64_t tiles_i, tiles_j;
};

__device__ __forceinline__ void query_span(int64_t t, int64_t window, int64_t* lo, int64_t* hi) {
    *hi = t + 1;
    *lo = window != 0 && t + 1 > window ? t + 1 - window : 0;
}

__device__ __forceinline__ void key_span(int64_t j, int64_t n, int64_t window, int64_t G, int64_t* lo, int64_t* hi) {
    *lo = j * G;
    const int64_t t_hi = window != 0 && j + window - 1 < n - 1 ? j + window - 1 : n - 1;
    *hi = (t_hi + 1) * G;
}

// The steps row r takes: [lo, hi). Rows past I take none.
__device__ __forceinline__ void row_span(const TileParams& p, int64_t r, int64_t n, int64_t I, int64_t* lo,
                                         int64_t* hi) {
    if (r >= I) {
        *lo = *hi = 0;
    } else if (p.mask == kMaskQueryRows) {
        query_span(r, p.window, lo, hi);
    } else if (p.mask == kMaskKeyRows) {
        key_span(r, n, p.window, p.group, lo, hi);
    } else {
        *lo = 0;
        *hi = p.L;
    }
}

// B arrives as floats and is widened to double once, when its stage is written to LDS: each of the 4 lanes of a wave
// (and the 4 waves) that read a B value takes it ready, and the inner loop has no conversions.
// CJ = 1, 2, 4: a workgroup covers 64 CJ columns, a lane 4 CJ of them; CJ = 0: 32 columns, a lane 2 of them (small
// grids: half the multiply-adds per step and twice the workgroups).
template <int CJ>
constexpr int tile_cols() {
    return CJ == 0 ? 32 : 64 * CJ;
}

template <int CJ>
constexpr int lane_cols() {
    return CJ == 0 ? 2 : 4 * CJ;
}

template <int CJ>
struct Stage {
    double a[kChunk][kTileRows];
    double b[kChunk][tile_cols<CJ>()];
};

template <int CJ>
constexpr int stage_copies() {
    return CJ == 0 ? 3 : 2 + 2 * CJ;
}

// Waits until at most `pending` of this wave's vector-memory operations are outstanding and its LDS writes have
// landed, then joins the workgroup.
template <int kPending>
__device__ __forceinline__ void wait_stage() {
    if (kPending == 0)
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kPending) : "memory");
}

__device__ __forceinline__ void workgroup_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Where the next stage's copies start, as wave-uniform values (scalar registers): step l, A's row of step l (from
// column i0), and B's row of query l / group (head 0 of the group; B rows are (query, head of the group) pairs) with
// rs = l % group. Each lane adds its own byte offsets.
struct StageCursor {
    int64_t l;
    const double* a;
    const float* b;
    int64_t rs;
};

// One stage's advance of the cursor, computed once per tile: A moves kChunk rows; B moves kChunk (query, head)
// pairs: kChunk / G queries, and one more when the head (rs + kChunk % G) wraps.
struct StageStep {
    int64_t a, b, b_carry, rs, group;
};

__device__ __forceinline__ StageStep stage_step(const Op& ao, const Op& bo) {
    StageStep t;
    t.group = bo.group;
    t.a = kChunk * ao.ld;
    t.b = (kChunk / bo.group) * bo.ld;
    t.b_carry = bo.ld;
    t.rs = kChunk % bo.group;
    return t;
}

// Advances the cursor by one stage with scalar arithmetic only.
__device__ __forceinline__ void advance(StageCursor& c, const StageStep& t) {
    c.l += kChunk;
    c.a += t.a;
    c.b += t.b;
    c.rs += t.rs;
    if (c.rs >= t.group) {
        c.rs -= t.group;
        c.b += t.b_carry;
    }
}

// The per-lane constants of the copies: A's byte column and its row stride; B's byte columns (two float2 chunks
// per 64-column block: 2cg, 2cg + 1 and 32 + 2cg, 33 + 2cg, cg = the lane's position among the block's 16 lanes,
// so that the doubles 16 lanes write, and later read, are 256 contiguous bytes: no LDS bank conflicts), its row
// strides and the divisor of grouped rows.
struct LaneCopy {
    uint32_t a_col, a_ld8;
    uint32_t b_col[2], b_ld4, b_in4;
    uint32_t group, magic;  // x / group == (x * magic) >> 16 for the x < 32 used here
};

// The stage of steps c.l .. c.l + 15 (steps past `last` repeat step `last`; they are never used). Wave w copies A
// rows (steps) 4w .. 4w + 3 straight to LDS (doubles: two per instruction) and loads B rows 4w .. 4w + 3 into
// registers, which store_stage_b widens and writes once the current stage has been computed.
template <int CJ>
__device__ __forceinline__ void issue_stage(Stage<CJ>& st, const StageCursor& c, const LaneCopy& lc, int64_t last,
                                            int wave, int lane, float2 (&breg)[CJ == 0 ? 2 : 2 * CJ]) {
    const int64_t left = last - c.l;  // the stage's steps past this one repeat it
    const uint32_t d = static_cast<uint32_t>(left < kChunk ? left : kChunk);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t r = static_cast<uint32_t>(4 * wave + 2 * t + (lane >> 5));
        const uint32_t off = (r < d ? r : d) * lc.a_ld8 + lc.a_col;
        copy16_to_lds_s(c.a, off, &st.a[4 * wave + 2 * t][0]);
    }
    constexpr int kLanesPerRow = CJ == 0 ? 16 : 16 * CJ;
    constexpr int kRowsPerCopy = 64 / kLanesPerRow;
    const int sub = lane / kLanesPerRow;
    const char* b = reinterpret_cast<const char*>(c.b);
#pragma unroll
    for (int t = 0; t < (CJ == 0 ? 1 : CJ); ++t) {
        const uint32_t r = static_cast<uint32_t>(4 * wave + t * kRowsPerCopy + sub);
        const uint32_t rr = r < d ? r : d;
        uint32_t off;
        if (lc.group == 1) {
            off = rr * lc.b_ld4;
        } else {
            const uint32_t x = rr + static_cast<uint32_t>(c.rs), q = (x * lc.magic) >> 16;
            off = q * lc.b_ld4 + (x - q * lc.group) * lc.b_in4;
        }
        breg[2 * t] = *reinterpret_cast<const float2*>(b + static_cast<uint64_t>(off + lc.b_col[0]));
        if (CJ != 0) breg[2 * t + 1] = *reinterpret_cast<const float2*>(b + static_cast<uint64_t>(off + lc.b_col[1]));
    }
}

template <int CJ>
__device__ __forceinline__ void store_stage_b(Stage<CJ>& st, int wave, int lane,
                                              const float2 (&breg)[CJ == 0 ? 2 : 2 * CJ]) {
    constexpr int kLanesPerRow = CJ == 0 ? 16 : 16 * CJ;
    constexpr int kRowsPerCopy = 64 / kLanesPerRow;
    const int sub = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int col = 64 * (q >> 4) + 2 * (q & 15);
#pragma unroll
    for (int t = 0; t < (CJ == 0 ? 1 : CJ); ++t) {
        double* row = &st.b[4 * wave + t * kRowsPerCopy + sub][0];
        *reinterpret_cast<double2*>(row + col) = double2{breg[2 * t].x, breg[2 * t].y};
        if (CJ != 0) *reinterpret_cast<double2*>(row + col + 32) = double2{breg[2 * t + 1].x, breg[2 * t + 1].y};
    }
}

// A lane's register tile: 4 consecutive rows (4 rg .. 4 rg + 3 of the wave's 16, rg = lane / 16) by 4 CJ columns
// (per 64-column block c: 64 c + 2 cg, + 1, 64 c + 32 + 2 cg, + 1; cg = lane % 16). Per step a lane reads its 4 A
// values (two 16-byte LDS reads shared by 16 lanes) and its 4 CJ B values (2 CJ 16-byte reads, 16 lanes reading 256
// contiguous bytes): 32 + 16 CJ bytes per lane for 16 CJ multiply-adds.
template <int CJ>
__device__ __forceinline__ int64_t tile_column(int c, int cg) {
    if (CJ == 0) return 2 * cg + c;
    return 64 * (c >> 2) + ((c & 2) ? 32 : 0) + 2 * cg + (c & 1);
}

template <int CJ>
__device__ __forceinline__ void read_step(const Stage<CJ>& st, int k, int wave, int rg, int cg, double (&a)[4],
                                          double (&b)[lane_cols<CJ>()]) {
    const double2* ar = reinterpret_cast<const double2*>(&st.a[k][wave * 16 + 4 * rg]);
    const double2 a01 = ar[0], a23 = ar[1];
    a[0] = a01.x;
    a[1] = a01.y;
    a[2] = a23.x;
    a[3] = a23.y;
    if (CJ == 0) {
        const double2 b01 = *reinterpret_cast<const double2*>(&st.b[k][2 * cg]);
        b[0] = b01.x;
        b[1] = b01.y;
        return;
    }
#pragma unroll
    for (int c = 0; c < CJ; ++c) {
        const double2 b01 = *reinterpret_cast<const double2*>(&st.b[k][64 * c + 2 * cg]);
        const double2 b23 = *reinterpret_cast<const double2*>(&st.b[k][64 * c + 32 + 2 * cg]);
        b[4 * c] = b01.x;
        b[4 * c + 1] = b01.y;
        b[4 * c + 2] = b23.x;
        b[4 * c + 3] = b23.y;
    }
}

// One step on the lane's tile: each product rounded, then added (the reference's multiply, then add).
template <int CJ>
__device__ __forceinline__ void step_tile(double (&acc)[4][lane_cols<CJ>()], const double (&a)[4], const double (&b)[lane_cols<CJ>()]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < lane_cols<CJ>(); ++c) {
            const double prod = a[i] * b[c];
            acc[i][c] = acc[i][c] + prod;
        }
}

// A full stage (every row takes every step), the next step's operands read while the current step computes.
template <int CJ>
__device__ __forceinline__ void stage_all(const Stage<CJ>& st, int wave, int rg, int cg, double (&acc)[4][lane_cols<CJ>()]) {
    double a[4], b[lane_cols<CJ>()];
    read_step<CJ>(st, 0, wave, rg, cg, a, b);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        double an[4], bn[lane_cols<CJ>()];
        if (k + 1 < kChunk) read_step<CJ>(st, k + 1, wave, rg, cg, an, bn);
        step_tile<CJ>(acc, a, b);
        if (k + 1 < kChunk) {
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = an[i];
#pragma unroll
            for (int c = 0; c < lane_cols<CJ>(); ++c) b[c] = bn[c];
        }
    }
}

// The wave's rows (tw + q, q < 16) that take step l, as a bit mask: the spans are intervals whose ends grow with the
// row, so the rows taking l are one run of q, from the span formulas of row_span. `t` is l / group (key rows: the
// query of step l), kept by the caller.
__device__ __forceinline__ uint32_t rows_taking(const TileParams& p, int64_t l, int64_t t, int64_t tw, int64_t I) {
    int64_t qa = 0, qb = (I - tw < 16 ? I - tw : 16) - 1;  // rows q in [qa, qb]
    if (p.mask == kMaskQueryRows) {  // l < t + 1, and l >= t + 1 - window
        qa = l - tw > qa ? l - tw : qa;
        if (p.window != 0) qb = l - tw + p.window - 1 < qb ? l - tw + p.window - 1 : qb;
    } else if (p.mask == kMaskKeyRows) {  // l >= j G, and (windowed) l / G < j + window
        qb = t - tw < qb ? t - tw : qb;
        if (p.window != 0) qa = t - tw - p.window + 1 > qa ? t - tw - p.window + 1 : qa;
    } else if (l >= p.L) {
        return 0u;
    }
    if (qa > qb) return 0u;
    const uint32_t upto = qb >= 31 ? 0xffffffffu : (2u << qb) - 1u;
    return upto & ~((1u << qa) - 1u);
}

// Steps l0 .. l0 + n - 1 of a stage, each taken by the rows whose span holds it (the lane's rows: bits 4 rg .. 4 rg + 3
// of the wave's mask). The query of a step (key rows) advances with it, one division per stage; the next step's
// operands are read while the current one computes.
template <int CJ>
__device__ __forceinline__ void stage_masked(const TileParams& p, const Stage<CJ>& st, int wave, int rg, int cg,
                                             int64_t l0, int n, int64_t tw, int64_t I, double (&acc)[4][lane_cols<CJ>()]) {
    const uint32_t G = p.mask == kMaskKeyRows ? static_cast<uint32_t>(p.group) : 1u;
    uint32_t t = static_cast<uint32_t>(l0) / G;  // steps of one (window, head) stay below 2^31
    uint32_t r = static_cast<uint32_t>(l0) - t * G;
    double a[4], b[lane_cols<CJ>()];
    read_step<CJ>(st, 0, wave, rg, cg, a, b);
    for (int k = 0; k < n; ++k) {
        double an[4], bn[lane_cols<CJ>()];
        read_step<CJ>(st, k + 1 < n ? k + 1 : k, wave, rg, cg, an, bn);
        const uint32_t take = __builtin_amdgcn_readfirstlane(rows_taking(p, l0 + k, t, tw, I));
        const uint32_t mine = take >> (4 * rg);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if ((mine >> i) & 1u) {
#pragma unroll
                for (int c = 0; c < lane_cols<CJ>(); ++c) {
                    const double prod = a[i] * b[c];
                    acc[i][c] = acc[i][c] + prod;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
#pragma unroll
        for (int c = 0; c < lane_cols<CJ>(); ++c) b[c] = bn[c];
        if (++r == G) {
            r = 0;
            ++t;
        }
    }
}

template <int CJ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(CJ <= 1 ? 4 : 2))) void attn_tile_kernel(
    TileParams p) {
    __shared__ __align__(16) Stage<CJ> st[2];
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    // block -> (rank by work, column tile, set, z): the longest reductions go first
    int64_t id = blockIdx.x;
    const int64_t zs = p.Z * p.sets;
    const int64_t zz = id % zs;
    id /= zs;
    const int64_t tj = id % p.tiles_j;
    const int64_t rank = id / p.tiles_j;
    const int64_t ti = p.mask == kMaskQueryRows ? p.tiles_i - 1 - rank : rank;
    const int set = static_cast<int>(zz / p.Z);
    const int64_t z = zz % p.Z;
    const OperandSet& o = p.set[set];
    const int64_t w = z / p.heads, hz = z % p.heads;
    const int64_t seg_w = uniform64(p.seg[w]), n = uniform64(p.seg[w + 1]) - seg_w;
    const int64_t I = p.rows_kind == 0 ? n : p.head_dim;
    const int64_t J = p.cols_kind == 0 ? n : p.head_dim;
    const int64_t i0 = ti * kTileRows, j0 = tj * tile_cols<CJ>();
    if (i0 >= I || j0 >= J) return;
    // spans are intervals whose ends grow with the row: the tile's steps are [lo(first row), hi(last row)), and the
    // steps every row of this wave takes are [lo(its last row), hi(its first row))
    int64_t t_lo, t_hi, w_lo, w_hi, dummy;
    row_span(p, i0, n, I, &t_lo, &dummy);
    row_span(p, (i0 + kTileRows - 1 < I ? i0 + kTileRows - 1 : I - 1), n, I, &dummy, &t_hi);
    const int64_t tw = i0 + wave * 16;
    if (tw < I) {
        row_span(p, tw, n, I, &dummy, &w_hi);
        row_span(p, (tw + 15 < I ? tw + 15 : I - 1), n, I, &w_lo, &dummy);
    } else {
        w_lo = w_hi = 0;
    }
    LaneCopy lc;
    lc.a_col = static_cast<uint32_t>((lane & 31) * 16);
    lc.a_ld8 = static_cast<uint32_t>(o.A.ld * 8);
    {
        const int q = lane % (CJ == 0 ? 16 : 16 * CJ);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t col = j0 + 64 * (q >> 4) + 32 * h + 2 * (q & 15);
            lc.b_col[h] = static_cast<uint32_t>((col + 2 <= p.b_row_alloc ? col : p.b_row_alloc - 2) * 4);
        }
    }
    lc.b_ld4 = static_cast<uint32_t>(o.B.ld * 4);
    lc.b_in4 = static_cast<uint32_t>(o.B.ld_inner * 4);
    lc.group = static_cast<uint32_t>(o.B.group);
    lc.magic = (65536u + lc.group - 1) / lc.group;
    StageCursor cur;
    cur.l = t_lo;
    cur.a = op_base<double>(o.A, w, seg_w, hz) + t_lo * o.A.ld + i0;
    cur.rs = t_lo % o.B.group;
    cur.b = op_base<float>(o.B, w, seg_w, hz) + (t_lo / o.B.group) * o.B.ld;
    const int rg = lane >> 4, cg = lane & 15;
    double acc[4][lane_cols<CJ>()];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int c = 0; c < lane_cols<CJ>(); ++c) acc[q][c] = 0.0;
    const int64_t steps = t_hi - t_lo;
    const int64_t stages = steps > 0 ? (steps + kChunk - 1) / kChunk : 0;
    const int64_t last = t_hi - 1;
    float2 breg[CJ == 0 ? 2 : 2 * CJ];
    if (stages > 0) {
        issue_stage<CJ>(st[0], cur, lc, last, wave, lane, breg);
        store_stage_b<CJ>(st[0], wave, lane, breg);
    }
    const StageStep step = stage_step(o.A, o.B);
    for (int64_t s = 0; s < stages; ++s) {
        if (s + 1 < stages) {
            advance(cur, step);
            issue_stage<CJ>(st[(s + 1) & 1], cur, lc, last, wave, lane, breg);
            wait_stage<stage_copies<CJ>()>();
        } else {
            wait_stage<0>();
        }
        const int64_t l0 = t_lo + s * kChunk;
        const int n_steps = static_cast<int>(t_hi - l0 < kChunk ? t_hi - l0 : kChunk);
        if (n_steps == kChunk && l0 >= w_lo && l0 + kChunk <= w_hi)
            stage_all<CJ>(st[s & 1], wave, rg, cg, acc);
        else
            stage_masked<CJ>(p, st[s & 1], wave, rg, cg, l0, n_steps, tw, I, acc);
        // the next stage's B, widened, into the other buffer (last read two stages ago, before the last barrier)
        if (s + 1 < stages) store_stage_b<CJ>(st[(s + 1) & 1], wave, lane, breg);
        workgroup_barrier();  // every wave is done with this stage before the next issue refills it
    }
    // the output rows' base and stride, opaque so the compiler keeps no per-element addresses across the reduction
    float* c_base = static_cast<float*>(const_cast<void*>(o.C.ptr)) + w * o.C.w_stride + seg_w * o.C.seg_stride +
                    (hz / o.C.head_div) * o.C.head_stride + tw * o.C.ld + j0;
    int64_t c_ld = o.C.ld;
    asm volatile("" : "+s"(c_base), "+s"(c_ld));
    const auto c_out = global_ptr(c_base);
    const double* rs = p.rowscale ? p.rowscale + z * p.rowscale_zstride + tw : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * rg + i;
        if (tw + q >= I) break;
        const double scale = rs ? rs[q] : 1.0;
#pragma unroll
        for (int c = 0; c < lane_cols<CJ>(); ++c) {
            const int64_t jl = tile_column<CJ>(c, cg);
            if (j0 + jl >= J) continue;
            double v = acc[i][c];
            if (rs) v = v * scale;
            c_out[q * c_ld + jl] = static_cast<float>(v);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The scores and dP (float x float, exact products) on the FP64 matrix cores.
//
// v_mfma_f64_16x16x4_f64 adds its four products to the accumulator as four FMAs in ascending k, each rounded: one
// instruction per 4 consecutive l is the serial chain over l = 0 .. head_dim - 1 that the vector FMAs computed
// (head_dim is a multiple of 4, so no step is padded). 64 rows
// (keys) x 256 columns (queries); the 4 waves sit side by side along the columns, each owning 64 x 64 outputs as
// 4 x 4 MFMA blocks. A stage is 16 l: A as [l / 4][row][l % 4] (one 16-byte copy per thread) and B as [l][column]
// (four per thread).
typedef double ma_v4d __attribute__((ext_vector_type(4)));
constexpr int kMfmaChunk = 16;

// B rows are padded by 16 floats so the four l rows a wave reads at once (lanes 16k .. 16k + 15 read row k) start
// in different banks.
constexpr int kMfmaBRow = 256 + 16;

struct MfmaStage {
    float a[kMfmaChunk * kTileRows];  // [l / 4][row][l % 4]
    float b[kMfmaChunk * kMfmaBRow];  // [l][column]
};

// The copies: a wave-uniform base (SGPRs) plus this lane's byte offset, computed once per tile, so a stage's copies
// cost the matrix core no vector instructions. Rows past the tile repeat its last row; in a last, partial stage
// (L % 16 != 0) the offsets are pulled back so every read stays inside the operand rows (those values are unused).
struct MfmaOffsets {
    uint32_t a, b[4];
};

__device__ __forceinline__ MfmaOffsets mfma_offsets(int64_t a_ld, int64_t i0, int64_t I, int64_t b_ld, int64_t j0,
                                                    int64_t b_row_alloc, int tid) {
    MfmaOffsets o;
    const int c = tid >> 6, ii = tid & 63;  // A copy: chunk c (l = 4c .. 4c + 3) of tile row ii
    const int64_t row = i0 + ii < I ? i0 + ii : I - 1;
    o.a = static_cast<uint32_t>((row * a_ld + 4 * c) * 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {  // B copy t: row r (l), 16-byte column chunk cc
        const int id = t * 256 + tid;
        const int r = id >> 6, cc = id & 63;
        const int64_t col = j0 + cc * 4 <= b_row_alloc - 4 ? j0 + cc * 4 : b_row_alloc - 4;
        o.b[t] = static_cast<uint32_t>((r * b_ld + col) * 4);
    }
    return o;
}

// Stage l .. l + 15 of A (row chunks, l < a_row_alloc) and B (rows l .. min(l + 15, L - 1)).
__device__ __forceinline__ void mfma_issue(MfmaStage& st, const float* A, int64_t a_row_alloc, const float* B,
                                           int64_t b_ld, const MfmaOffsets& o, int64_t l, int64_t L, int tid,
                                           int wave) {
    const bool full = l + kMfmaChunk <= L;
    uint32_t va = o.a;
    if (!full) {
        const int64_t over = l + 4 * (tid >> 6) - (a_row_alloc - 4);
        if (over > 0) va -= static_cast<uint32_t>(over * 4);
    }
    copy16_to_lds_s(A + l, va, &st.a[wave * 64 * 4]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint32_t vb = o.b[t];
        if (!full) {
            const int64_t over = l + ((t * 256 + tid) >> 6) - (L - 1);
            if (over > 0) vb -= static_cast<uint32_t>(over * b_ld * 4);
        }
        copy16_to_lds_s(B + l * b_ld, vb, &st.b[(4 * t + wave) * kMfmaBRow]);  // row 4t + wave
    }
}

__device__ __forceinline__ void mfma_frags(const MfmaStage& st, int s, int wave, int lane, double (&a)[4],
                                           double (&b)[4]) {
    const int k = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        a[q] = static_cast<double>(st.a[(s * kTileRows + 16 * q + c16) * 4 + k]);
        b[q] = static_cast<double>(st.b[(4 * s + k) * kMfmaBRow + wave * 64 + 16 * q + c16]);
    }
}

__device__ __forceinline__ void mfma_4x4(const double (&a)[4], const double (&b)[4], ma_v4d (&acc)[4][4]) {
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            acc[bi][bj] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[bi], b[bj], acc[bi][bj], 0, 0, 0);
}

template <bool kOutDouble>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_mfma_kernel(TileParams p) {
    __shared__ MfmaStage st[2];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    int64_t id = blockIdx.x;
    const int64_t zz = id % p.Z;
    id /= p.Z;
    const int64_t tj = id % p.tiles_j;
    const int64_t ti = id / p.tiles_j;
    const OperandSet& o = p.set[0];
    const int64_t w = zz / p.heads, hz = zz % p.heads;
    const int64_t seg_w = p.seg[w], n = p.seg[w + 1] - seg_w;
    const int64_t I = p.rows_kind == 0 ? n : p.head_dim;
    const int64_t J = p.cols_kind == 0 ? n : p.head_dim;
    const int64_t i0 = ti * kTileRows, j0 = tj * 256;
    if (i0 >= I || j0 >= J) return;
    if (p.mask == kMaskTileCausal) {  // score tiles no query sees: every key row above every query column
        if (i0 > j0 + 255) return;
        if (p.window != 0 && i0 + kTileRows - 1 + p.window - 1 < j0) return;
    }
    const float* A = op_base<float>(o.A, w, seg_w, hz);
    const float* B = op_base<float>(o.B, w, seg_w, hz);
    ma_v4d acc[4][4];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj) acc[bi][bj] = ma_v4d{0.0, 0.0, 0.0, 0.0};
    const int64_t L = p.L;
    const int64_t stages = (L + kMfmaChunk - 1) / kMfmaChunk;
    const MfmaOffsets off = mfma_offsets(o.A.ld, i0, I, o.B.ld, j0, p.b_row_alloc, tid);
    mfma_issue(st[0], A, p.a_row_alloc, B, o.B.ld, off, 0, L, tid, wave);
    for (int64_t s = 0; s < stages; ++s) {
        if (s + 1 < stages) {
            mfma_issue(st[(s + 1) & 1], A, p.a_row_alloc, B, o.B.ld, off, (s + 1) * kMfmaChunk, L, tid, wave);
            wait_stage<5>();
        } else {
            wait_stage<0>();
        }
        // 4-l steps of this stage (L is a multiple of 4); the fragments of step k + 1 are read during step k
        const int steps = static_cast<int>((L - s * kMfmaChunk < kMfmaChunk ? L - s * kMfmaChunk : kMfmaChunk) / 4);
        double a[4], b[4];
        mfma_frags(st[s & 1], 0, wave, lane, a, b);
#pragma unroll
        for (int k = 0; k < kMfmaChunk / 4; ++k) {
            if (k < steps) {
                double an[4], bn[4];
                if (k + 1 < kMfmaChunk / 4 && k + 1 < steps) mfma_frags(st[s & 1], k + 1, wave, lane, an, bn);
                mfma_4x4(a, b, acc);
                if (k + 1 < kMfmaChunk / 4 && k + 1 < steps)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        a[q] = an[q];
                        b[q] = bn[q];
                    }
            }
        }
        workgroup_barrier();  // every wave is done with this stage before the next issue refills it
    }
    const int64_t elem = kOutDouble ? 8 : 4;
    char* c_base = reinterpret_cast<char*>(const_cast<void*>(o.C.ptr)) +
                   (w * o.C.w_stride + seg_w * o.C.seg_stride + (hz / o.C.head_div) * o.C.head_stride) * elem;
    int64_t c_ld = o.C.ld * elem;
    asm volatile("" : "+s"(c_base), "+s"(c_ld));  // no output addresses kept live across the reduction
    const auto c_out = global_ptr(c_base);
    const double* rs = p.rowscale ? p.rowscale + zz * p.rowscale_zstride : nullptr;
    const int64_t jw = j0 + wave * 64 + (lane & 15);
    if constexpr (kOutDouble) {
        // the largest score of this 64-key tile each query sees (visible keys only; NaN scores skipped, -inf when
        // none): the softmax takes its maximum from these instead of a walk over the scores
        if (p.tile_max) {
            const auto tm = global_ptr(p.tile_max + zz * p.tile_max_zstride + (i0 / 64) * p.tile_max_ld);
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int64_t t = jw + 16 * bj;
                double m = -__builtin_huge_val();
#pragma unroll
                for (int bi = 0; bi < 4; ++bi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t i = i0 + 16 * bi + (lane >> 4) + 4 * r;
                        const bool seen = i < I && t < J &&
                                          (p.mask != kMaskTileCausal || (i <= t && (p.window == 0 || t - i < p.window)));
                        const double v = acc[bi][bj][r] * p.out_scale;
                        if (seen && v > m) m = v;
                    }
                const double m16 = __shfl_xor(m, 16, 64);
                m = m16 > m ? m16 : m;
                const double m32 = __shfl_xor(m, 32, 64);
                m = m32 > m ? m32 : m;
                if ((lane >> 4) == 0 && t < J) tm[t] = m;
            }
        }
    }
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t i = i0 + 16 * bi + (lane >> 4) + 4 * r;
            if (i >= I) continue;
            const auto row = c_out + i * c_ld;
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int64_t j = jw + 16 * bj;
                if (j >= J) continue;
                if constexpr (kOutDouble) {
                    reinterpret_cast<global_pointer<double>>(row)[j] = acc[bi][bj][r] * p.out_scale;
                } else {
                    double v = acc[bi][bj][r];
                    if (rs) v = v * rs[i];
                    reinterpret_cast<global_pointer<float>>(row)[j] = static_cast<float>(v);
                }
            }
        }
}

Op op_of(const AttnOperand& o) {
    return Op{o.ptr, o.w_stride, o.seg_stride, o.head_stride, o.head_div > 0 ? o.head_div : 1, o.ld, o.ld_inner,
              o.group > 0 ? o.group : 1};
}

}  // namespace

int launch_attn_tiles(const AttnTileCall& c, hipStream_t stream) {
    TileParams p{};
    p.sets = c.second ? 2 : 1;
    p.set[0] = OperandSet{op_of(c.A), op_of(c.B), op_of(c.C)};
    p.set[1] = c.second ? OperandSet{op_of(c.A2), op_of(c.B2), op_of(c.C2)} : p.set[0];
    p.rowscale = c.rowscale;
    p.rowscale_zstride = c.rowscale_zstride;
    p.out_scale = c.out_scale;
    p.tile_max = c.tile_max;
    p.tile_max_zstride = c.tile_max_zstride;
    p.tile_max_ld = c.tile_max_ld;
    if (c.tile_max)
        DLLM_REQUIRE(c.a_float && c.out_double && (c.mask == kMaskTileCausal || c.mask == kMaskNone) &&
                         c.rows_kind == 0 && c.cols_kind == 0,
                     "tile maxima are for the scores (keys x queries)");
    p.seg = c.seg;
    p.heads = c.heads;
    p.Z = c.windows * c.heads;
    p.rows_kind = c.rows_kind;
    p.cols_kind = c.cols_kind;
    p.head_dim = c.head_dim;
    p.group = c.group > 0 ? c.group : 1;
    p.window = c.window;
    p.L = c.L;
    p.mask = c.mask;
    const int64_t I = c.rows_kind == 0 ? c.max_len : c.head_dim;
    const int64_t J = c.cols_kind == 0 ? c.max_len : c.head_dim;
    const int cj = c.cols_per_lane;
    p.b_row_alloc = c.b_row_alloc > 0 ? c.b_row_alloc : J;
    p.a_row_alloc = c.a_row_alloc;
    p.tiles_i = static_cast<int64_t>(ceil_div(I, kTileRows));
    p.tiles_j = static_cast<int64_t>(ceil_div(J, cj == 0 ? 32 : 64 * cj));
    DLLM_REQUIRE(cj == 0 || cj == 1 || cj == 2 || cj == 4, "attention tiles are 64 rows x 32, 64, 128 or 256 columns");
    DLLM_REQUIRE(p.b_row_alloc % 4 == 0 && p.b_row_alloc >= J, "attention operand rows must hold whole 16-byte chunks");
    if (c.a_float)
        DLLM_REQUIRE(c.exact_products && cj == 4 && c.mask != kMaskQueryRows && c.mask != kMaskKeyRows &&
                         p.a_row_alloc % 4 == 0 && p.a_row_alloc >= c.L && c.A.ld % 4 == 0,
                     "float A operands are the scores' K or V rows (exact products over head_dim)");
    else
        DLLM_REQUIRE(c.A.ld % 2 == 0 && c.A.ld >= static_cast<int64_t>(round_up(static_cast<size_t>(I), kTileRows)),
                     "attention double operand rows must be padded to whole 64-row tiles");
    const int64_t blocks = p.tiles_i * p.tiles_j * p.Z * p.sets;
    if (blocks == 0) return kOk;
    DLLM_REQUIRE(blocks < (int64_t{1} << 31), "attention matmul grid too large");
    const dim3 grid(static_cast<unsigned>(blocks));
    if (c.a_float) {
        DLLM_REQUIRE(c.L % 4 == 0 && c.B.group <= 1 && c.A.group <= 1 && !c.second,
                     "the matrix-core scores take whole 4-l steps and plain operand rows");
        if (c.out_double)
            hipLaunchKernelGGL(attn_mfma_kernel<true>, dim3(static_cast<unsigned>(p.tiles_i * p.tiles_j * p.Z)),
                               dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(attn_mfma_kernel<false>, dim3(static_cast<unsigned>(p.tiles_i * p.tiles_j * p.Z)),
                               dim3(256), 0, stream, p);
    } else {
        DLLM_REQUIRE(!c.exact_products && !c.out_double,
                     "double A operands are the probability and dS rows (multiply, then add; float outputs)");
        if (cj == 2) hipLaunchKernelGGL(attn_tile_kernel<2>, grid, dim3(256), 0, stream, p);
        else if (cj == 1) hipLaunchKernelGGL(attn_tile_kernel<1>, grid, dim3(256), 0, stream, p);
        else if (cj == 0) hipLaunchKernelGGL(attn_tile_kernel<0>, grid, dim3(256), 0, stream, p);
        else return fail(kInvalidArgument, "double A operands take 32, 64 or 128 columns per tile");
    }
    return check_launch("attention tiles");
}

}  // namespace dllm_hip
