// Launchers of the training step's attention: batched matmuls (attn_lds.hip) and per-query chains (attn_chains.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dllm_hip {

// The `window` of the chain launchers that makes every key visible to every query (no causal mask).
constexpr int64_t kAllKeys = -1;

enum AttnMask {
    kMaskNone = 0,
    kMaskQueryRows = 1,   // rows are queries t; reduce over the keys t sees, ascending
    kMaskKeyRows = 2,     // rows are keys j; reduce over (query, head of the group) pairs that see j, ascending
    kMaskTileCausal = 3,  // output [key][query] tiles nothing can see are skipped (scores, dP)
};

// Where operand rows live for batch entry z = (window w, head hz):
// base = ptr + w * w_stride + seg[w] * seg_stride + (hz / head_div) * head_stride, row(l) = (l / group) * ld +
// (l % group) * ld_inner (elements of the operand's type).
struct AttnOperand {
    const void* ptr = nullptr;
    int64_t w_stride = 0, seg_stride = 0, head_stride = 0, head_div = 1;
    int64_t ld = 0, ld_inner = 0, group = 1;
};

// One attention matmul (attn_lds.hip) over every (window, head) z = w * heads + hz of a step:
// C[i][j] = sum over l in row i's span, ascending, of A[l][i] * B[l][j], times a row scale or a constant.
// A is double [L][rows padded to 64] (products multiply-then-add, float output, 64 or 128 columns per tile) or, for
// the scores and dP, float rows A[i][l] read transposed (a_float: exact products, 256 columns per tile). `second`
// runs a second matmul of the same shape in the same launch (dk and dv).
struct AttnTileCall {
    AttnOperand A, B, C;
    bool second = false;
    AttnOperand A2, B2, C2;
    const double* rowscale = nullptr;  // float outputs: row multiplier before rounding, [z][row]
    int64_t rowscale_zstride = 0;
    const int64_t* seg = nullptr;  // device window offsets
    int64_t windows = 0, heads = 0, max_len = 0, head_dim = 0, group = 1, window = 0, L = 0;
    int rows_kind = 0, cols_kind = 0;  // 0: window positions, 1: head_dim
    int mask = kMaskNone;
    int cols_per_lane = 4;    // 1, 2 or 4: a workgroup covers 64 x cols_per_lane columns; 0: 32 columns
    int64_t b_row_alloc = 0;  // floats readable per B row from column 0 (multiple of 4, >= J); 0: J
    bool a_float = false;
    int64_t a_row_alloc = 0;  // a_float: floats readable in each A row (multiple of 4, >= L)
    bool exact_products = true;  // float x float products: fused multiply-add is exact
    bool out_double = false;
    double out_scale = 1.0;
    // scores only: tile_max[z * tile_max_zstride + (key / 64) * tile_max_ld + query] = the largest score of that
    // 64-key tile the query sees (visible keys; NaN skipped; -inf when none)
    double* tile_max = nullptr;
    int64_t tile_max_zstride = 0, tile_max_ld = 0;
};

int launch_attn_tiles(const AttnTileCall& c, hipStream_t stream);

#ifndef DLLM_ATTN_NARROW_BELOW
#define DLLM_ATTN_NARROW_BELOW 1024
#endif
// cols_per_lane of a head_dim-wide multiply-add output (out, dq, dk/dv) over `rows` rows of `heads` heads in
// `windows` windows, `sets` matmuls per launch: 64-column tiles (their 4 x 4 register tiles leave room for four waves
// per SIMD, which keeps the vector ALU busier than wider tiles' A reuse), or 32-column tiles (0) when the 64-column
// grid would leave the chip short of workgroups: twice the workgroups, each step half the work.
inline int attn_value_cols(int64_t rows, int64_t head_dim, int64_t heads, int64_t windows, int64_t sets) {
    const int64_t workgroups = (rows + 63) / 64 * ((head_dim + 63) / 64) * heads * windows * sets;
    return workgroups < DLLM_ATTN_NARROW_BELOW ? 0 : 1;
}
// The forward softmax chains over S^T in place (E^T and inv). With tile maxima (the scores' tile_max, same z and ld
// layout as there) the maximum comes from them and the scores are walked once; without, twice.
int launch_softmax_rows(double* st, int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                        int64_t max_len, int64_t window, double* inv, int64_t inv_zstride, hipStream_t stream,
                        const double* tile_max = nullptr, int64_t tile_max_zstride = 0, int64_t tile_max_ld = 0);
// The softmax backward (grad.hpp:262-278): D per query (dvec: windows * heads * inv_zstride doubles of workspace),
// then ds written over dpt and p, ds in the key-row layout of dk / dv:
// pg / dsg[w][g][(t * group + hh)][j] (dst_ld per row, dst_zstride per (window, kv head)).
int launch_dsoftmax_regroup(const double* et, double* dpt, int64_t ld, int64_t zstride, const int64_t* seg,
                            int64_t windows, int64_t heads, int64_t group, int64_t max_len, int64_t window,
                            const double* inv, int64_t inv_zstride, double scale, double* dvec, double* pg,
                            double* dsg, int64_t dst_ld, int64_t dst_zstride, hipStream_t stream,
                            const double* slope = nullptr);
// Soft-capped scores (Gemma 2; grad.hpp:247-251 and nn.hpp:539-541): every one of `count` scaled scores s becomes
// cap t with t = tanh(s / cap), and slope gets 1 - t t (the backward's factor), in double.
int launch_softcap_scores(double* st, double* slope, int64_t count, double cap, hipStream_t stream);
int launch_heads_transpose(const float* src, int64_t row_stride, int64_t head_dim, void* dst, bool to_double,
                           int64_t ld, int64_t zstride, const int64_t* seg, int64_t windows, int64_t heads,
                           int64_t max_len, hipStream_t stream);

}  // namespace dllm_hip
