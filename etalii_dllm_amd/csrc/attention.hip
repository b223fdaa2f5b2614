// Causal grouped-query attention, forward and backward, with the reference's per-row orders
// (cpp/include/dllm/nn.hpp:535-615 and grad.hpp:206-301).
//
// A (query t, head h) row is one wave. Scores of its visible keys are computed by the lanes (one key per lane at a
// time, the head_dim dot in ascending order as exact float products, so fused multiply-add is legal there), staged
// in LDS as doubles; the max is a first-maximum reduction (ties keep the lowest key, as the serial scan does); the
// exponentials are parallel; the totals and the backward's D are serial double chains on lane 0; the value and
// query-gradient sums run over keys in ascending order with one accumulator per output dimension per lane, as an
// unfused multiply and add (the probability is not a float, so the product rounds).
//
// The backward is two passes. Pass A (query-stationary) recomputes p exactly, forms dp, D and ds, writes dq and
// stores p and ds per (row, key) in the workspace. Pass B (key-stationary) gives each (key j, kv head g) one wave
// that sums dk[j] += ds * q and dv[j] += p * dout over the queries t ascending and, for each t, the heads of group g
// ascending: the (t, h) visiting order of the reference's double accumulators.
#include "common.h"
#include "devmath.h"
#include "kernels.h"

namespace dllm_hip {

namespace {

struct Span {
    int64_t first, count;
};

// attention_span (nn.hpp:733-748) for sequence-local query t.
__device__ __forceinline__ Span span_of(int64_t t, int64_t kv_len, int causal, int64_t q_offset, int64_t window) {
    const int64_t pos = q_offset + t;
    if (!causal) {
        if (window == 0) return {0, kv_len};
        const int64_t f = pos + 1 > window ? pos + 1 - window : 0;
        const int64_t last = pos + window < kv_len ? pos + window : kv_len;
        return {f, last > f ? last - f : 0};
    }
    const int64_t end = pos + 1 < kv_len ? pos + 1 : kv_len;
    const int64_t f = window != 0 && end > window ? end - window : 0;
    return {f, end - f};
}

// Locates packed row `row` (of total rows = sum q_len * q_heads) in its sequence.
struct RowRef {
    int seq;
    int64_t t, h;  // sequence-local query, head
};

__device__ __forceinline__ RowRef locate(const AttentionBatch& b, int64_t q_heads, int64_t packed_q) {
    // packed_q is the packed query index; sequences are few, a linear scan is cheap and uniform.
    int s = 0;
    while (s + 1 < b.count && packed_q >= b.q_start[s + 1]) ++s;
    return {s, packed_q - b.q_start[s], 0};
}

// s_j = f32-exact dot(q, k_j) * scale (+ softcap), for keys first .. first+count-1, into sc[0..count).
__device__ __forceinline__ void scores(const float* __restrict__ qh, const float* __restrict__ kbase, int64_t kstride,
                                       int64_t head_dim, double scale, double softcap, int64_t count, double* sc,
                                       double* slope, int lane) {
    for (int64_t j = lane; j < count; j += 64) {
        const float* kj = kbase + j * kstride;
        double d = 0.0;
        for (int64_t i = 0; i < head_dim; ++i)
            d = __builtin_fma(static_cast<double>(qh[i]), static_cast<double>(kj[i]), d);
        double sj = d * scale;
        double sl = 1.0;
        if (softcap > 0.0) {
            const double th = dtanh(sj / softcap);
            sj = softcap * th;
            sl = 1.0 - th * th;
        }
        sc[j] = sj;
        if (slope) slope[j] = sl;
    }
}

// First maximum of sc[0..count) (the serial `if (s > max) max = s` scan), reduced over the wave.
__device__ __forceinline__ double first_max(const double* sc, int64_t count, int lane) {
    double best = 0.0;
    int64_t bi = -1;
    for (int64_t j = lane; j < count; j += 64) {
        const double v = sc[j];
        if (bi < 0 || v > best) {
            best = v;
            bi = j;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const double ov = __shfl_xor(best, off, 64);
        const int64_t oi = __shfl_xor(bi, off, 64);
        bool take;
        if (bi < 0) take = oi >= 0;
        else if (oi < 0) take = false;
        else if (ov > best) take = true;
        else if (best > ov) take = false;
        else take = oi < bi;
        if (take) {
            best = ov;
            bi = oi;
        }
    }
    return __shfl(best, 0, 64);
}

// Forward (nn.hpp:535-569, 574-615). The row's scores are staged in dynamic LDS (max_kv doubles per wave) or, for key
// lengths past kMaxKvLds, in the row's slice of `stage` (max_kv doubles per (query, head) row).
__global__ __launch_bounds__(64) void attention_forward_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                               const float* __restrict__ v, float* __restrict__ out,
                                                               AttentionShape sh, AttentionBatch b, double* stage) {
    extern __shared__ double lds[];
    double* sc = stage ? stage + static_cast<int64_t>(blockIdx.x) * b.max_kv : lds;
    const int lane = threadIdx.x;
    const int64_t packed_q = blockIdx.x / sh.q_heads;
    const int64_t h = blockIdx.x % sh.q_heads;
    const RowRef ref = locate(b, sh.q_heads, packed_q);
    const int64_t qlen = b.q_len[ref.seq], kvlen = b.kv_len[ref.seq];
    if (ref.t >= qlen) return;
    const int64_t group = sh.q_heads / sh.kv_heads, g = h / group;
    const Span sp = span_of(ref.t, kvlen, sh.causal, sh.q_offset, sh.window);
    float* oh = out + (packed_q * sh.q_heads + h) * sh.value_dim;
    if (sp.count == 0) {
        for (int64_t i = lane; i < sh.value_dim; i += 64) oh[i] = 0.0f;
        return;
    }
    const int64_t kv0 = b.kv_start[ref.seq] + sp.first;
    const float* qh = q + (packed_q * sh.q_heads + h) * sh.head_dim;
    scores(qh, k + (kv0 * sh.kv_heads + g) * sh.head_dim, sh.kv_heads * sh.head_dim, sh.head_dim, sh.scale,
           sh.softcap, sp.count, sc, nullptr, lane);
    __syncthreads();
    const double mx = first_max(sc, sp.count, lane);
    for (int64_t j = lane; j < sp.count; j += 64) sc[j] = dexp(sc[j] - mx);
    __syncthreads();
    double total = 0.0;
    if (lane == 0)
        for (int64_t j = 0; j < sp.count; ++j) total += sc[j];
    total = __shfl(total, 0, 64);
    const double inv = 1.0 / total;
    const float* vb = v + (kv0 * sh.kv_heads + g) * sh.value_dim;
    const int64_t vstride = sh.kv_heads * sh.value_dim;
    for (int64_t i = lane; i < sh.value_dim; i += 64) {
        double acc = 0.0;
        for (int64_t j = 0; j < sp.count; ++j) acc += sc[j] * static_cast<double>(vb[j * vstride + i]);
        oh[i] = static_cast<float>(acc * inv);
    }
}

// Pass A of the backward (grad.hpp:221-292 per row): dq, plus p and ds per visible key into the workspace rows
// (indexed by sequence-local key), for pass B. Staging: 3 * max_kv doubles of dynamic LDS, or (key lengths past
// kMaxKvLds) the row's 3 * max_kv doubles of `stage`.
__global__ __launch_bounds__(64) void attention_backward_rows_kernel(const float* __restrict__ q,
                                                                     const float* __restrict__ k,
                                                                     const float* __restrict__ v,
                                                                     const float* __restrict__ dout,
                                                                     float* __restrict__ dq, double* __restrict__ P,
                                                                     double* __restrict__ DS, AttentionShape sh,
                                                                     AttentionBatch b, double* stage) {
    extern __shared__ double lds[];
    const int lane = threadIdx.x;
    double* base = stage ? stage + static_cast<int64_t>(blockIdx.x) * 3 * b.max_kv : lds;
    double* pr = base;                 // scores, then probabilities
    double* dpr = base + b.max_kv;     // dp, then ds
    double* slope = base + 2 * b.max_kv;
    const int64_t packed_q = blockIdx.x / sh.q_heads;
    const int64_t h = blockIdx.x % sh.q_heads;
    const RowRef ref = locate(b, sh.q_heads, packed_q);
    const int64_t qlen = b.q_len[ref.seq], kvlen = b.kv_len[ref.seq];
    if (ref.t >= qlen) return;
    const int64_t group = sh.q_heads / sh.kv_heads, g = h / group;
    const Span sp = span_of(ref.t, kvlen, sh.causal, sh.q_offset, sh.window);
    const int64_t row = packed_q * sh.q_heads + h;
    float* dqh = dq + row * sh.head_dim;
    if (sp.count == 0) {
        for (int64_t i = lane; i < sh.head_dim; i += 64) dqh[i] = 0.0f;
        return;
    }
    const int64_t kv0 = b.kv_start[ref.seq] + sp.first;
    const float* qh = q + row * sh.head_dim;
    const float* doh = dout + row * sh.value_dim;
    const float* kb = k + (kv0 * sh.kv_heads + g) * sh.head_dim;
    const float* vb = v + (kv0 * sh.kv_heads + g) * sh.value_dim;
    const int64_t kstride = sh.kv_heads * sh.head_dim, vstride = sh.kv_heads * sh.value_dim;
    scores(qh, kb, kstride, sh.head_dim, sh.scale, sh.softcap, sp.count, pr, slope, lane);
    __syncthreads();
    const double mx = first_max(pr, sp.count, lane);
    for (int64_t j = lane; j < sp.count; j += 64) pr[j] = dexp(pr[j] - mx);
    __syncthreads();
    double total = 0.0;
    if (lane == 0)
        for (int64_t j = 0; j < sp.count; ++j) total += pr[j];
    total = __shfl(total, 0, 64);
    const double inv = 1.0 / total;
    for (int64_t j = lane; j < sp.count; j += 64) {
        pr[j] *= inv;
        const float* vj = vb + j * vstride;
        double d = 0.0;
        for (int64_t i = 0; i < sh.value_dim; ++i)
            d = __builtin_fma(static_cast<double>(doh[i]), static_cast<double>(vj[i]), d);
        dpr[j] = d;
    }
    __syncthreads();
    double weighted = 0.0;
    if (lane == 0)
        for (int64_t j = 0; j < sp.count; ++j) weighted += pr[j] * dpr[j];
    weighted = __shfl(weighted, 0, 64);
    double* prow = P + row * b.max_kv;
    double* dsrow = DS + row * b.max_kv;
    for (int64_t j = lane; j < sp.count; j += 64) {
        const double ds = pr[j] * (dpr[j] - weighted) * slope[j] * sh.scale;
        dpr[j] = ds;
        prow[sp.first + j] = pr[j];
        dsrow[sp.first + j] = ds;
    }
    __syncthreads();
    for (int64_t i = lane; i < sh.head_dim; i += 64) {
        double acc = 0.0;
        for (int64_t j = 0; j < sp.count; ++j) acc += dpr[j] * static_cast<double>(kb[j * kstride + i]);
        dqh[i] = static_cast<float>(acc);
    }
}

// Pass B (grad.hpp:277-289, 295-300): one wave per (sequence, key j, kv head g).
__global__ __launch_bounds__(64) void attention_backward_keys_kernel(const float* __restrict__ q,
                                                                     const float* __restrict__ dout,
                                                                     const double* __restrict__ P,
                                                                     const double* __restrict__ DS,
                                                                     float* __restrict__ dk, float* __restrict__ dv,
                                                                     AttentionShape sh, AttentionBatch b) {
    const int lane = threadIdx.x;
    const int64_t packed_kv = blockIdx.x / sh.kv_heads;
    const int64_t g = blockIdx.x % sh.kv_heads;
    int s = 0;
    while (s + 1 < b.count && packed_kv >= b.kv_start[s + 1]) ++s;
    const int64_t j = packed_kv - b.kv_start[s];
    const int64_t qlen = b.q_len[s], kvlen = b.kv_len[s];
    if (j >= kvlen) return;
    const int64_t group = sh.q_heads / sh.kv_heads;
    const int64_t q0 = b.q_start[s];
    for (int64_t i = lane; i < sh.head_dim || i < sh.value_dim; i += 64) {
        double dka = 0.0, dva = 0.0;
        for (int64_t t = 0; t < qlen; ++t) {
            const Span sp = span_of(t, kvlen, sh.causal, sh.q_offset, sh.window);
            if (j < sp.first || j >= sp.first + sp.count) continue;
            for (int64_t hh = 0; hh < group; ++hh) {
                const int64_t row = (q0 + t) * sh.q_heads + g * group + hh;
                const double ds = DS[row * b.max_kv + j];
                const double p = P[row * b.max_kv + j];
                if (i < sh.head_dim) dka += ds * static_cast<double>(q[row * sh.head_dim + i]);
                if (i < sh.value_dim) dva += p * static_cast<double>(dout[row * sh.value_dim + i]);
            }
        }
        if (i < sh.head_dim) dk[(packed_kv * sh.kv_heads + g) * sh.head_dim + i] = static_cast<float>(dka);
        if (i < sh.value_dim) dv[(packed_kv * sh.kv_heads + g) * sh.value_dim + i] = static_cast<float>(dva);
    }
}

constexpr int64_t kMaxKvLds = 2048;  // LDS staging up to here (pass A: 3 doubles per key, 48 KB)

size_t rows_of(const AttentionShape& s) { return static_cast<size_t>(s.q_len) * static_cast<size_t>(s.q_heads); }

}  // namespace

size_t attention_stage_bytes(const AttentionShape& s, const AttentionBatch& b, bool backward) {
    if (b.max_kv <= kMaxKvLds) return 0;
    return rows_of(s) * static_cast<size_t>(b.max_kv) * sizeof(double) * (backward ? 3 : 1);
}

int launch_attention(const float* q, const float* k, const float* v, float* out, const AttentionShape& s,
                     const AttentionBatch& b, void* stage, hipStream_t stream) {
    DLLM_REQUIRE(s.kv_heads > 0 && s.q_heads % s.kv_heads == 0, "q_heads must be a multiple of kv_heads");
    DLLM_REQUIRE(b.max_kv <= kMaxKvLds || stage != nullptr, "attention past 2048 keys needs its staging workspace");
    const int64_t total_q = s.q_len;  // packed queries of all sequences
    if (total_q == 0 || s.q_heads == 0) return kOk;
    const bool in_lds = b.max_kv <= kMaxKvLds;
    const size_t lds = in_lds ? static_cast<size_t>(b.max_kv > 0 ? b.max_kv : 1) * sizeof(double) : 0;
    hipLaunchKernelGGL(attention_forward_kernel, dim3(static_cast<unsigned>(total_q * s.q_heads)), dim3(64), lds,
                       stream, q, k, v, out, s, b, in_lds ? nullptr : static_cast<double*>(stage));
    return check_launch("attention");
}

size_t attention_backward_workspace(const AttentionShape& s, const AttentionBatch& b, int64_t total_q) {
    return static_cast<size_t>(total_q) * static_cast<size_t>(s.q_heads) * static_cast<size_t>(b.max_kv > 0 ? b.max_kv : 1) *
           sizeof(double) * 2;
}

int launch_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                              float* dv, const AttentionShape& s, const AttentionBatch& b, int64_t total_q,
                              int64_t total_kv, void* workspace, void* stage, hipStream_t stream) {
    DLLM_REQUIRE(s.kv_heads > 0 && s.q_heads % s.kv_heads == 0, "q_heads must be a multiple of kv_heads");
    DLLM_REQUIRE(b.max_kv <= kMaxKvLds || stage != nullptr, "attention past 2048 keys needs its staging workspace");
    double* P = static_cast<double*>(workspace);
    double* DS = P + static_cast<size_t>(total_q) * s.q_heads * (b.max_kv > 0 ? b.max_kv : 1);
    if (total_q > 0 && s.q_heads > 0) {
        const bool in_lds = b.max_kv <= kMaxKvLds;
        const size_t lds = in_lds ? static_cast<size_t>(b.max_kv > 0 ? b.max_kv : 1) * sizeof(double) * 3 : 0;
        hipLaunchKernelGGL(attention_backward_rows_kernel, dim3(static_cast<unsigned>(total_q * s.q_heads)), dim3(64),
                           lds, stream, q, k, v, dout, dq, P, DS, s, b, in_lds ? nullptr : static_cast<double*>(stage));
        DLLM_TRY(check_launch("attention_backward_rows"));
    }
    if (total_kv > 0 && s.kv_heads > 0) {
        hipLaunchKernelGGL(attention_backward_keys_kernel, dim3(static_cast<unsigned>(total_kv * s.kv_heads)), dim3(64),
                           0, stream, q, dout, P, DS, dk, dv, s, b);
        DLLM_TRY(check_launch("attention_backward_keys"));
    }
    return kOk;
}

}  // namespace dllm_hip
