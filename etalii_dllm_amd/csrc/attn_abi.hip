// The kernel-level attention entry points on the training step's matrix-core path, for self-attention shapes
// (q_len == kv_len = n, no cached prefix, no soft-cap, head_dim == value_dim, a multiple of 4): causal with an
// optional sliding window, or every key visible. One sequence, laid out as the step lays out one window:
//   S^T[h][j][t] = sum_i k[j][i] q[t][i], times scale     (FP64 matrix cores: exact float products, ascending i)
//   the softmax chains per query over its keys ascending   (first maximum, e = exp(s - max), serial total, 1 / total)
//   out[t] = f32((sum_j e v_j) inv_t)                       (multiply-then-add tiles, keys ascending)
// and the backward:
//   dP^T = V dout^T; D_t = sum_j p dp; ds = p (dp - D_t) scale; dq = sum_j ds k_j; dk_j = sum over (t, head of the
//   group) of ds q; dv_j = sum of p dout
// in the orders of nn.hpp:535-615 and grad.hpp:206-301. Other shapes take the row kernels of attention.hip.
#include "attn_step.h"
#include "common.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

__global__ void self_seg_kernel(int64_t* seg, int64_t n) {
    if (threadIdx.x == 0) {
        seg[0] = 0;
        seg[1] = n;
    }
}

struct SelfLayout {
    int64_t n = 0, Tp = 0, nh = 0, nkv = 0, hd = 0, G = 1;
    size_t seg = 0, qt = 0, et = 0, inv = 0, tmax = 0, forward = 0;
    size_t dot = 0, dpt = 0, dvec = 0, pg = 0, dsg = 0, backward = 0;
};

SelfLayout self_layout(size_t n, size_t nh, size_t nkv, size_t hd) {
    SelfLayout L;
    L.n = static_cast<int64_t>(n);
    L.Tp = static_cast<int64_t>(round_up(n > 0 ? n : 1, 64));
    L.nh = static_cast<int64_t>(nh);
    L.nkv = static_cast<int64_t>(nkv > 0 ? nkv : 1);
    L.hd = static_cast<int64_t>(hd);
    L.G = L.nh / L.nkv;
    const size_t Tp = static_cast<size_t>(L.Tp), sq = nh * Tp * Tp * sizeof(double);
    size_t off = 0;
    const auto take = [&](size_t bytes) {
        const size_t at = off;
        off += round_up(bytes > 0 ? bytes : 1, 256);
        return at;
    };
    L.seg = take(2 * sizeof(int64_t));
    L.qt = take(nh * hd * Tp * sizeof(float));
    L.et = take(sq);
    L.inv = take(nh * Tp * sizeof(double));
    L.tmax = take(nh * (Tp / 64) * Tp * sizeof(double));
    L.forward = off;
    L.dot = take(nh * hd * Tp * sizeof(float));
    L.dpt = take(sq);
    L.dvec = take(nh * Tp * sizeof(double));
    L.pg = take(sq);
    L.dsg = take(sq);
    L.backward = off;
    return L;
}

template <typename T>
T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

// The chains' window argument: the sliding window of a causal call (0 = every earlier key), or every key.
int64_t chain_window(int causal, int64_t window) { return causal ? window : kAllKeys; }

AttnTileCall base_call(const SelfLayout& L, const int64_t* seg, int causal, int64_t window) {
    AttnTileCall c;
    c.seg = seg;
    c.windows = 1;
    c.heads = L.nh;
    c.max_len = L.n;
    c.head_dim = L.hd;
    c.group = L.G;
    c.window = causal ? window : 0;
    return c;
}

// S^T = K Q^T scale, then E^T and inv (the forward's probabilities, in place).
int self_probabilities(const float* q, const float* k, const SelfLayout& L, double scale, int causal, int64_t window,
                       void* ws, hipStream_t s) {
    int64_t* seg = at<int64_t>(ws, L.seg);
    float* qt = at<float>(ws, L.qt);
    double* et = at<double>(ws, L.et);
    const int64_t QD = L.nh * L.hd, KVD = L.nkv * L.hd;
    hipLaunchKernelGGL(self_seg_kernel, dim3(1), dim3(64), 0, s, seg, L.n);
    DLLM_TRY(check_launch("attention segments"));
    DLLM_TRY(launch_heads_transpose(q, QD, L.hd, qt, false, L.Tp, L.hd * L.Tp, seg, 1, L.nh, L.n, s));
    AttnTileCall g = base_call(L, seg, causal, window);
    g.A = AttnOperand{k, 0, KVD, L.hd, L.G, KVD, 0, 1};
    g.a_float = true;
    g.a_row_alloc = L.hd;
    g.B = AttnOperand{qt, L.nh * L.hd * L.Tp, 0, L.hd * L.Tp, 1, L.Tp, 0, 1};
    g.C = AttnOperand{et, L.nh * L.Tp * L.Tp, 0, L.Tp * L.Tp, 1, L.Tp, 0, 1};
    g.rows_kind = 0;
    g.cols_kind = 0;
    g.L = L.hd;
    g.mask = causal ? kMaskTileCausal : kMaskNone;
    g.cols_per_lane = 4;
    g.b_row_alloc = L.Tp;
    g.exact_products = true;
    g.out_double = true;
    g.out_scale = scale;
    g.tile_max = at<double>(ws, L.tmax);
    g.tile_max_zstride = (L.Tp / 64) * L.Tp;
    g.tile_max_ld = L.Tp;
    DLLM_TRY(launch_attn_tiles(g, s));
    return launch_softmax_rows(et, L.Tp, L.Tp * L.Tp, seg, 1, L.nh, L.n, chain_window(causal, window),
                               at<double>(ws, L.inv), L.Tp, s, g.tile_max, g.tile_max_zstride, g.tile_max_ld);
}

// C[t] = sum over the keys t sees of A[j][t] B[j] (multiply, then add), into [n][heads][hd] rows.
AttnTileCall query_sum(const SelfLayout& L, const int64_t* seg, int causal, int64_t window, const double* A,
                       const float* B, float* C) {
    const int64_t QD = L.nh * L.hd, KVD = L.nkv * L.hd;
    AttnTileCall c = base_call(L, seg, causal, window);
    c.A = AttnOperand{A, L.nh * L.Tp * L.Tp, 0, L.Tp * L.Tp, 1, L.Tp, 0, 1};
    c.B = AttnOperand{B, 0, KVD, L.hd, L.G, KVD, 0, 1};
    c.C = AttnOperand{C, 0, QD, L.hd, 1, QD, 0, 1};
    c.rows_kind = 0;
    c.cols_kind = 1;
    c.L = causal ? 0 : L.n;
    c.mask = causal ? kMaskQueryRows : kMaskNone;
    c.cols_per_lane = attn_value_cols(L.n, L.hd, L.nh, 1, 1);
    c.exact_products = false;
    c.out_double = false;
    return c;
}

}  // namespace

bool self_attention_fast(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads, size_t head_dim,
                         size_t value_dim, int causal, int64_t q_offset, size_t window, double softcap) {
    const bool offset_zero = q_offset < 0 || q_offset == 0;
    return q_len == kv_len && q_len > 0 && q_len <= 65535 && offset_zero && softcap == 0.0 && kv_heads > 0 &&
           q_heads % kv_heads == 0 && head_dim == value_dim && head_dim > 0 && head_dim % 4 == 0 &&
           (causal || window == 0);
}

size_t self_attention_workspace(size_t n, size_t q_heads, size_t kv_heads, size_t head_dim, bool backward) {
    const SelfLayout L = self_layout(n, q_heads, kv_heads, head_dim);
    return backward ? L.backward : L.forward;
}

int self_attention_forward(const float* q, const float* k, const float* v, float* out, size_t n, size_t q_heads,
                           size_t kv_heads, size_t head_dim, double scale, int causal, int64_t window, void* ws,
                           hipStream_t s) {
    const SelfLayout L = self_layout(n, q_heads, kv_heads, head_dim);
    DLLM_TRY(self_probabilities(q, k, L, scale, causal, window, ws, s));
    AttnTileCall o = query_sum(L, at<int64_t>(ws, L.seg), causal, window, at<double>(ws, L.et), v, out);
    o.rowscale = at<double>(ws, L.inv);
    o.rowscale_zstride = L.Tp;
    return launch_attn_tiles(o, s);
}

int self_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                            float* dv, size_t n, size_t q_heads, size_t kv_heads, size_t head_dim, double scale,
                            int causal, int64_t window, void* ws, hipStream_t s) {
    const SelfLayout L = self_layout(n, q_heads, kv_heads, head_dim);
    DLLM_TRY(self_probabilities(q, k, L, scale, causal, window, ws, s));
    const int64_t* seg = at<int64_t>(ws, L.seg);
    double* et = at<double>(ws, L.et);
    double* dpt = at<double>(ws, L.dpt);
    double* pg = at<double>(ws, L.pg);
    double* dsg = at<double>(ws, L.dsg);
    float* dot = at<float>(ws, L.dot);
    const int64_t QD = L.nh * L.hd, KVD = L.nkv * L.hd, Tp = L.Tp, G = L.G;
    DLLM_TRY(launch_heads_transpose(dout, QD, L.hd, dot, false, Tp, L.hd * Tp, seg, 1, L.nh, L.n, s));
    // dP^T[j][t] = sum_i v[j][i] dout[t][i]
    AttnTileCall g = base_call(L, seg, causal, window);
    g.A = AttnOperand{v, 0, KVD, L.hd, G, KVD, 0, 1};
    g.a_float = true;
    g.a_row_alloc = L.hd;
    g.B = AttnOperand{dot, L.nh * L.hd * Tp, 0, L.hd * Tp, 1, Tp, 0, 1};
    g.C = AttnOperand{dpt, L.nh * Tp * Tp, 0, Tp * Tp, 1, Tp, 0, 1};
    g.rows_kind = 0;
    g.cols_kind = 0;
    g.L = L.hd;
    g.mask = causal ? kMaskTileCausal : kMaskNone;
    g.cols_per_lane = 4;
    g.b_row_alloc = Tp;
    g.exact_products = true;
    g.out_double = true;
    g.out_scale = 1.0;
    DLLM_TRY(launch_attn_tiles(g, s));
    // D, p = e inv and ds = p (dp - D) scale: ds over dP^T (dq's operand), p and ds in the key-row layout
    // [g][(t, hh)][j] of dk and dv
    const int64_t gz = Tp * G * Tp;
    DLLM_TRY(launch_dsoftmax_regroup(et, dpt, Tp, Tp * Tp, seg, 1, L.nh, G, L.n, chain_window(causal, window),
                                     at<double>(ws, L.inv), Tp, scale, at<double>(ws, L.dvec), pg, dsg, Tp, gz, s));
    // dq[t] = sum_j ds[t][j] k[j]
    DLLM_TRY(launch_attn_tiles(query_sum(L, seg, causal, window, dpt, k, dq), s));
    // dk[j] = sum over (t, hh) of ds q; dv[j] = sum of p dout; one launch
    AttnTileCall kc = base_call(L, seg, causal, window);
    kc.heads = L.nkv;
    kc.A = AttnOperand{dsg, L.nkv * gz, 0, gz, 1, Tp, 0, 1};
    kc.B = AttnOperand{q, 0, QD, G * L.hd, 1, QD, L.hd, G};
    kc.C = AttnOperand{dk, 0, KVD, L.hd, 1, KVD, 0, 1};
    kc.second = true;
    kc.A2 = AttnOperand{pg, L.nkv * gz, 0, gz, 1, Tp, 0, 1};
    kc.B2 = AttnOperand{dout, 0, QD, G * L.hd, 1, QD, L.hd, G};
    kc.C2 = AttnOperand{dv, 0, KVD, L.hd, 1, KVD, 0, 1};
    kc.rows_kind = 0;
    kc.cols_kind = 1;
    kc.L = causal ? 0 : L.n * G;
    kc.mask = causal ? kMaskKeyRows : kMaskNone;
    kc.cols_per_lane = attn_value_cols(L.n, L.hd, L.nkv, 1, 2);
    kc.exact_products = false;
    kc.out_double = false;
    return launch_attn_tiles(kc, s);
}

}  // namespace dllm_hip
