// The kernel-level C ABI (include/dllm_hip.h): argument checks in the reference binding's terms
// (cpp/kernels.cpp), workspace carving, and one launch sequence per entry point.
#include <string.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "common.h"
#include "devmath.h"
#include "dllm_hip.h"
#include "kernels.h"
#include "workspace.h"

using namespace dllm_hip;

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

size_t linear_ws(size_t rows, size_t in, size_t out) {
    Layout l;
    l.add<double>(in * static_cast<size_t>(padded_rows(rows)));  // x^T as double
    l.add<float>(in * out);                                         // W^T
    return l.bytes;
}

size_t linear_backward_ws(size_t rows, size_t in, size_t out) {
    Layout l;
    l.add<double>(rows * static_cast<size_t>(padded_rows(out)));  // dy as double [rows][out_pad]
    l.add<double>(out * static_cast<size_t>(padded_rows(rows)));  // dy^T as double [out][rows_pad]
    return l.bytes;
}

struct AttnBatchStorage {
    int64_t v[4];
};

}  // namespace

extern "C" {

const char* dllm_hip_last_error(void) { return last_error(); }
const char* dllm_hip_version(void) { return "dllm_hip 0.1 (gfx950)"; }

int dllm_hip_device_count(int* count) { return check_hip(hipGetDeviceCount(count), "hipGetDeviceCount"); }
int dllm_hip_alloc(void** p, size_t bytes) { return check_hip(hipMalloc(p, bytes > 0 ? bytes : 1), "hipMalloc"); }
int dllm_hip_release(void* p) { return check_hip(hipFree(p), "hipFree"); }
int dllm_hip_upload(void* dst, const void* src, size_t bytes) {
    return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "upload");
}
int dllm_hip_download(void* dst, const void* src, size_t bytes) {
    return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "download");
}
int dllm_hip_memset(void* p, int value, size_t bytes) { return check_hip(hipMemset(p, value, bytes), "memset"); }
int dllm_hip_synchronize(void) { return check_hip(hipDeviceSynchronize(), "synchronize"); }
int dllm_hip_copy(void* dst, const void* src, size_t bytes, void* stream) {
    return launch_device_copy(dst, src, bytes, static_cast<hipStream_t>(stream));
}

namespace {
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

size_t dllm_hip_linear_workspace(size_t rows, size_t in, size_t out) { return linear_ws(rows, in, out); }

// rope_inv_freq (numerics.py:267-349): the default frequencies exp(-(2i / dim) log theta) with the portable exp and
// log, then the scaling, every step in the Python code's double operation order (its ints divide as correctly
// rounded doubles; min, max, floor and ceil as written).
int dllm_hip_rope_inv_freq(size_t head_dim, double theta, size_t rotary_dim, const dllm_hip_rope_scaling* sc,
                           double* out) {
    const size_t dim = rotary_dim == 0 ? head_dim : rotary_dim;
    DLLM_REQUIRE(dim > 0 && dim % 2 == 0 && dim <= head_dim, "rotary_dim must be even, positive and at most head_dim");
    DLLM_REQUIRE(out != nullptr, "null output");
    const int64_t kind = sc ? sc->kind : 0;
    DLLM_REQUIRE(kind >= 0 && kind <= 4, "unsupported rope scaling kind");
    DLLM_REQUIRE(kind != 3 || sc->factors != nullptr, "longrope needs its factors");
    const size_t pairs = dim / 2;
    const double log_theta = dlog(theta);
    for (size_t i = 0; i < pairs; ++i)
        out[i] = dexp(-(static_cast<double>(2 * i) / static_cast<double>(dim)) * log_theta);
    const double pi = 3.141592653589793;  // math.pi
    if (kind == 1) {  // linear: positions divided by the factor
        for (size_t i = 0; i < pairs; ++i) out[i] = out[i] / sc->factor;
    } else if (kind == 2) {  // llama3
        const double low = sc->low_freq_factor, high = sc->high_freq_factor;
        const double original = sc->original_max_position_embeddings;
        const double low_freq_wavelen = original / low, high_freq_wavelen = original / high;
        for (size_t i = 0; i < pairs; ++i) {
            const double f = out[i];
            const double wavelen = 2 * pi / f;
            if (wavelen < high_freq_wavelen) continue;
            if (wavelen > low_freq_wavelen) {
                out[i] = f / sc->factor;
            } else {
                const double smooth = (original / wavelen - low) / (high - low);
                out[i] = (1 - smooth) * f / sc->factor + smooth * f;
            }
        }
    } else if (kind == 3) {  // longrope: each frequency divided by its factor (the chosen short or long set)
        for (size_t i = 0; i < pairs; ++i) out[i] = out[i] / sc->factors[i];
    } else if (kind == 4) {  // yarn (_yarn, numerics.py:325-349)
        const double d = static_cast<double>(dim), original = sc->original_max_position_embeddings;
        double low = d * dlog(original / (sc->beta_fast * 2 * pi)) / (2 * log_theta);
        double high = d * dlog(original / (sc->beta_slow * 2 * pi)) / (2 * log_theta);
        if (sc->truncate) {
            low = std::floor(low);
            high = std::ceil(high);
        }
        if (low < 0) low = 0;
        if (high > d - 1) high = d - 1;
        if (low == high) high += 0.001;
        for (size_t i = 0; i < pairs; ++i) {
            double ramp = (static_cast<double>(i) - low) / (high - low);
            ramp = std::min(std::max(ramp, 0.0), 1.0);  // 0: extrapolate, 1: interpolate
            const double f = out[i];
            out[i] = f / sc->factor * ramp + f * (1 - ramp);
        }
    }
    return kOk;
}

int dllm_hip_linear(const float* x, const float* w, const float* bias, float* out, size_t rows, size_t in, size_t out_f,
                    void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= linear_ws(rows, in, out_f), "workspace too small for linear");
    if (rows == 0 || out_f == 0) return kOk;
    Carve c(workspace, workspace_bytes);
    const int64_t R = static_cast<int64_t>(rows), K = static_cast<int64_t>(in), N = static_cast<int64_t>(out_f);
    double* xT = c.take<double>(K * padded_rows(R));
    float* wT = c.take<float>(K * N);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const hipStream_t s = as_stream(stream);
    DLLM_TRY(launch_transpose_f32(w, N, K, wT, s));
    GemmCall g;
    if (K % 4 == 0 && N % 4 == 0 && aligned16(x)) {  // the matmul reads x itself
        g.Af = x;
        g.a_kind = 2;
        g.lda = K;
    } else {
        DLLM_TRY(launch_to_double(x, R, K, K, nullptr, 0, xT, padded_rows(R), s));
        g.A = xT;
        g.lda = padded_rows(R);
    }
    g.B = wT;
    g.ldb = N;
    g.C = out;
    g.ldc = N;
    g.I = R;
    g.J = N;
    g.l0 = 0;
    g.l1 = K;
    g.bias = bias;
    return launch_gemm(g, s);
}

int dllm_hip_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t dim, double eps, int unit,
                      void* stream) {
    return launch_rms_norm(x, w, out, static_cast<int64_t>(rows), static_cast<int64_t>(dim), eps, unit, nullptr,
                           as_stream(stream));
}

size_t dllm_hip_rope_workspace(size_t tokens, size_t rotary_dim) {
    Layout l;
    l.add<double>(tokens * (rotary_dim / 2));
    l.add<double>(tokens * (rotary_dim / 2));
    return l.bytes;
}

int dllm_hip_rope(const float* x, const int64_t* positions, const double* inv_freq, float* out, size_t tokens,
                  size_t heads, size_t head_dim, size_t rotary_dim, int interleaved, int inverse, void* workspace,
                  size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(rotary_dim % 2 == 0 && rotary_dim <= head_dim, "2 * len(inv_freq) must not exceed head_dim");
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_rope_workspace(tokens, rotary_dim), "workspace too small for rope");
    Carve c(workspace, workspace_bytes);
    const int64_t half = static_cast<int64_t>(rotary_dim / 2);
    double* ct = c.take<double>(tokens * half);
    double* st = c.take<double>(tokens * half);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const hipStream_t s = as_stream(stream);
    if (half + static_cast<int64_t>(head_dim - rotary_dim) <= 64)
        return launch_rope_direct(x, positions, inv_freq, out, static_cast<int64_t>(tokens), static_cast<int64_t>(heads),
                                  static_cast<int64_t>(head_dim), static_cast<int64_t>(rotary_dim), interleaved,
                                  inverse, s);
    DLLM_TRY(launch_rope_tables(positions, static_cast<int64_t>(tokens), inv_freq, half, ct, st, s));
    return launch_rope(x, nullptr, ct, st, out, static_cast<int64_t>(tokens), static_cast<int64_t>(heads),
                       static_cast<int64_t>(head_dim), static_cast<int64_t>(rotary_dim), interleaved, inverse, s);
}

static int single_sequence(size_t q_len, size_t kv_len, void* ws, hipStream_t s, AttentionBatch* b) {
    const int64_t host[4] = {0, static_cast<int64_t>(q_len), 0, static_cast<int64_t>(kv_len)};
    int64_t* d = static_cast<int64_t*>(ws);
    DLLM_TRY(check_hip(hipMemcpyAsync(d, host, sizeof host, hipMemcpyHostToDevice, s), "attention upload"));
    // the host array must stay valid until the copy completes
    DLLM_TRY(check_hip(hipStreamSynchronize(s), "attention upload"));
    b->q_start = d;
    b->q_len = d + 1;
    b->kv_start = d + 2;
    b->kv_len = d + 3;
    b->count = 1;
    b->max_q = static_cast<int64_t>(q_len);
    b->max_kv = static_cast<int64_t>(kv_len);
    return kOk;
}

static int attention_shape(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads, size_t head_dim,
                           size_t value_dim, double scale, int causal, int64_t q_offset, size_t window, double softcap,
                           AttentionShape* sh) {
    DLLM_REQUIRE(kv_heads > 0 && q_heads % kv_heads == 0, "q heads must be a multiple of kv heads");
    if (q_offset < 0) q_offset = static_cast<int64_t>(kv_len) - static_cast<int64_t>(q_len);
    DLLM_REQUIRE(q_offset >= 0, "q_offset must be non-negative");
    *sh = AttentionShape{static_cast<int64_t>(q_len), static_cast<int64_t>(kv_len), static_cast<int64_t>(q_heads),
                         static_cast<int64_t>(kv_heads), static_cast<int64_t>(head_dim),
                         static_cast<int64_t>(value_dim), scale, causal, q_offset, static_cast<int64_t>(window),
                         softcap};
    return kOk;
}

// The row kernels' staging bytes for a call's shape (0 when every row's keys fit in LDS).
static size_t row_stage_bytes(size_t q_len, size_t kv_len, size_t q_heads, bool backward) {
    AttentionShape sh{};
    sh.q_len = static_cast<int64_t>(q_len);
    sh.q_heads = static_cast<int64_t>(q_heads);
    AttentionBatch b{};
    b.max_kv = static_cast<int64_t>(kv_len);
    return attention_stage_bytes(sh, b, backward);
}

size_t dllm_hip_attention_workspace(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads, size_t head_dim,
                                    size_t value_dim, int causal, int64_t q_offset, size_t window, double softcap) {
    if (self_attention_fast(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, causal, q_offset, window, softcap))
        return self_attention_workspace(q_len, q_heads, kv_heads, head_dim, false);
    Layout l;
    l.add<AttnBatchStorage>(1);
    l.add<char>(row_stage_bytes(q_len, kv_len, q_heads, false));
    return l.bytes;
}

int dllm_hip_attention(const float* q, const float* k, const float* v, float* out, size_t q_len, size_t kv_len,
                       size_t q_heads, size_t kv_heads, size_t head_dim, size_t value_dim, double scale, int causal,
                       int64_t q_offset, size_t window, double softcap, void* workspace, size_t workspace_bytes,
                       void* stream) {
    AttentionShape sh;
    DLLM_TRY(attention_shape(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, scale, causal, q_offset, window,
                             softcap, &sh));
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_attention_workspace(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim,
                                                                 causal, q_offset, window, softcap),
                 "workspace too small for attention");
    const hipStream_t s = as_stream(stream);
    if (self_attention_fast(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, causal, q_offset, window, softcap))
        return self_attention_forward(q, k, v, out, q_len, q_heads, kv_heads, head_dim, scale, causal,
                                      static_cast<int64_t>(window), workspace, s);
    Carve c(workspace, workspace_bytes);
    AttnBatchStorage* bs = c.take<AttnBatchStorage>(1);
    char* stage = c.take<char>(row_stage_bytes(q_len, kv_len, q_heads, false));
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    AttentionBatch b;
    DLLM_TRY(single_sequence(q_len, kv_len, bs, s, &b));
    return launch_attention(q, k, v, out, sh, b, stage, s);
}

int dllm_hip_silu(const float* x, float* out, size_t n, void* stream) {
    return launch_silu(x, out, static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_gelu_tanh(const float* x, float* out, size_t n, void* stream) {
    return launch_gelu_tanh(x, out, static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_softcap(const float* x, float* out, size_t n, double cap, void* stream) {
    DLLM_REQUIRE(cap > 0.0, "cap must be positive");
    return launch_softcap(x, out, static_cast<int64_t>(n), cap, as_stream(stream));
}

int dllm_hip_sigmoid_elementwise(const float* x, float* out, size_t n, void* stream) {
    return launch_sigmoid(x, out, static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_swiglu(const float* gate, const float* up, float* out, size_t n, int kind, void* stream) {
    DLLM_REQUIRE(kind == 0 || kind == 2, "kind must be silu (0) or gelu_tanh (2)");
    if (kind == 2) return launch_geglu_tanh(gate, up, out, static_cast<int64_t>(n), as_stream(stream));
    return launch_swiglu_forward(gate, up, nullptr, out, static_cast<int64_t>(n), as_stream(stream));
}

size_t dllm_hip_linear_backward_workspace(size_t rows, size_t in, size_t out) {
    return linear_backward_ws(rows, in, out);
}

int dllm_hip_linear_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                             size_t rows, size_t in, size_t out_f, void* workspace, size_t workspace_bytes,
                             void* stream) {
    DLLM_REQUIRE(workspace_bytes >= linear_backward_ws(rows, in, out_f), "workspace too small for linear_backward");
    Carve c(workspace, workspace_bytes);
    const int64_t R = static_cast<int64_t>(rows), K = static_cast<int64_t>(in), N = static_cast<int64_t>(out_f);
    double* dy_d = c.take<double>(R * padded_rows(N));
    double* dyT_d = c.take<double>(N * padded_rows(R));
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const hipStream_t s = as_stream(stream);
    // the matmuls read dy itself when its rows are whole 16-byte chunks; otherwise as doubles
    const bool float_dx = N % 4 == 0 && K % 4 == 0 && aligned16(dy) && aligned16(w);
    const bool float_dw = N % 4 == 0 && K % 4 == 0 && aligned16(dy) && aligned16(x);
    if ((dw && !float_dw) || (dx && !float_dx))
        DLLM_TRY(launch_to_double(dy, R, N, N, dw && !float_dw ? dy_d : nullptr, padded_rows(N),
                                  dx && !float_dx ? dyT_d : nullptr, padded_rows(R), s));
    if (dx) {
        if (N == 0) {
            DLLM_TRY(check_hip(hipMemsetAsync(dx, 0, sizeof(float) * R * K, s), "memset"));
        } else {
            GemmCall g;  // dx[r][k] = sum_n dy[r][n] w[n][k]
            if (float_dx) {
                g.Af = dy;
                g.a_kind = 2;
                g.lda = N;
            } else {
                g.A = dyT_d;
                g.lda = padded_rows(R);
            }
            g.B = w;
            g.ldb = K;
            g.C = dx;
            g.ldc = K;
            g.I = R;
            g.J = K;
            g.l0 = 0;
            g.l1 = N;
            DLLM_TRY(launch_gemm(g, s));
        }
    }
    if (dw) {
        if (R == 0) {
            DLLM_TRY(check_hip(hipMemsetAsync(dw, 0, sizeof(float) * N * K, s), "memset"));
        } else {
            GemmCall g;  // dw[n][k] = sum_r dy[r][n] x[r][k]
            if (float_dw) {
                g.Af = dy;
                g.a_kind = 1;
                g.lda = N;
            } else {
                g.A = dy_d;
                g.lda = padded_rows(N);
            }
            g.B = x;
            g.ldb = K;
            g.C = dw;
            g.ldc = K;
            g.I = N;
            g.J = K;
            g.l0 = 0;
            g.l1 = R;
            DLLM_TRY(launch_gemm(g, s));
        }
    }
    if (db) {
        const int64_t seg[2] = {0, R};
        DLLM_TRY(launch_column_sums(0, dy, nullptr, nullptr, N, seg, 1, nullptr, db, s));
    }
    return kOk;
}

size_t dllm_hip_rms_norm_backward_workspace(size_t rows) {
    Layout l;
    l.add<double>(rows);
    return l.bytes;
}

int dllm_hip_rms_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, size_t rows,
                               size_t dim, double eps, int unit, void* workspace, size_t workspace_bytes,
                               void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_rms_norm_backward_workspace(rows), "workspace too small");
    Carve c(workspace, workspace_bytes);
    double* inv = c.take<double>(rows);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const hipStream_t s = as_stream(stream);
    const int64_t R = static_cast<int64_t>(rows), D = static_cast<int64_t>(dim);
    DLLM_TRY(launch_rms_norm_backward_dx(x, w, dy, dx, nullptr, R, D, eps, unit, inv, s));
    if (dw) {
        const int64_t seg[2] = {0, R};
        DLLM_TRY(launch_column_sums(1, dy, x, inv, D, seg, 1, nullptr, dw, s));
    }
    return kOk;
}

int dllm_hip_silu_backward(const float* x, const float* dy, float* out, size_t n, void* stream) {
    return launch_silu_backward(x, dy, out, static_cast<int64_t>(n), as_stream(stream));
}

size_t dllm_hip_attention_backward_workspace(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                                             size_t head_dim, size_t value_dim, int causal, int64_t q_offset,
                                             size_t window, double softcap) {
    if (self_attention_fast(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, causal, q_offset, window, softcap))
        return self_attention_workspace(q_len, q_heads, kv_heads, head_dim, true);
    Layout l;
    l.add<AttnBatchStorage>(1);
    l.add<double>(2 * q_len * q_heads * std::max<size_t>(kv_len, 1));
    l.add<char>(row_stage_bytes(q_len, kv_len, q_heads, true));
    return l.bytes;
}

int dllm_hip_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq,
                                float* dk, float* dv, size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                                size_t head_dim, size_t value_dim, double scale, int causal, int64_t q_offset,
                                size_t window, double softcap, void* workspace, size_t workspace_bytes,
                                void* stream) {
    AttentionShape sh;
    DLLM_TRY(attention_shape(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, scale, causal, q_offset, window,
                             softcap, &sh));
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_attention_backward_workspace(q_len, kv_len, q_heads, kv_heads, head_dim,
                                                                          value_dim, causal, q_offset, window,
                                                                          softcap),
                 "workspace too small for attention_backward");
    const hipStream_t s = as_stream(stream);
    if (self_attention_fast(q_len, kv_len, q_heads, kv_heads, head_dim, value_dim, causal, q_offset, window, softcap))
        return self_attention_backward(q, k, v, dout, dq, dk, dv, q_len, q_heads, kv_heads, head_dim, scale, causal,
                                       static_cast<int64_t>(window), workspace, s);
    Carve c(workspace, workspace_bytes);
    AttnBatchStorage* bs = c.take<AttnBatchStorage>(1);
    double* pds = c.take<double>(2 * q_len * q_heads * std::max<size_t>(kv_len, 1));
    char* stage = c.take<char>(row_stage_bytes(q_len, kv_len, q_heads, true));
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    AttentionBatch b;
    DLLM_TRY(single_sequence(q_len, kv_len, bs, s, &b));
    return launch_attention_backward(q, k, v, dout, dq, dk, dv, sh, b, static_cast<int64_t>(q_len),
                                     static_cast<int64_t>(kv_len), pds, stage, s);
}

size_t dllm_hip_cross_entropy_workspace(size_t rows) {
    Layout l;
    l.add<double>(rows);
    l.add<double>(rows);
    l.add<double>(rows);
    l.add<int64_t>(2);
    l.add<double>(1);
    l.add<int>(1);
    return l.bytes;
}

int dllm_hip_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, size_t rows, size_t vocab,
                           double scale, double* loss, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_cross_entropy_workspace(rows), "workspace too small for cross_entropy");
    Carve c(workspace, workspace_bytes);
    double* rm = c.take<double>(rows);
    double* rt = c.take<double>(rows);
    double* rl = c.take<double>(rows);
    int64_t* seg = c.take<int64_t>(2);
    double* loss_d = c.take<double>(1);
    int* flag = c.take<int>(1);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const hipStream_t s = as_stream(stream);
    const int64_t host_seg[2] = {0, static_cast<int64_t>(rows)};
    DLLM_TRY(check_hip(hipMemcpyAsync(seg, host_seg, sizeof host_seg, hipMemcpyHostToDevice, s), "upload"));
    DLLM_TRY(check_hip(hipMemsetAsync(flag, 0, sizeof(int), s), "memset"));
    DLLM_TRY(launch_cross_entropy(logits, targets, dlogits, static_cast<int64_t>(rows), static_cast<int64_t>(vocab),
                                  scale, seg, 1, rm, rt, rl, loss_d, flag, s));
    double host_loss = 0.0;
    int host_flag = 0;
    DLLM_TRY(check_hip(hipMemcpyAsync(&host_loss, loss_d, sizeof host_loss, hipMemcpyDeviceToHost, s), "download"));
    DLLM_TRY(check_hip(hipMemcpyAsync(&host_flag, flag, sizeof host_flag, hipMemcpyDeviceToHost, s), "download"));
    DLLM_TRY(check_hip(hipStreamSynchronize(s), "cross_entropy"));
    if (host_flag) return fail(kInvalidArgument, "target out of range");
    if (loss) *loss = rows == 0 ? 0.0 : host_loss;
    return kOk;
}

size_t dllm_hip_embedding_backward_workspace(size_t rows) {
    Layout l;
    l.add<int64_t>(rows);      // order
    l.add<int64_t>(rows + 1);  // group starts
    l.add<int64_t>(rows);      // output row of each group
    return l.bytes;
}

int dllm_hip_embedding_backward(const float* dy, const int64_t* tokens, float* out, size_t rows, size_t dim,
                                size_t vocab, void* workspace, size_t workspace_bytes, void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_embedding_backward_workspace(rows), "workspace too small");
    const hipStream_t s = as_stream(stream);
    std::vector<int64_t> tok(rows);
    if (rows > 0) {
        DLLM_TRY(check_hip(hipMemcpyAsync(tok.data(), tokens, rows * sizeof(int64_t), hipMemcpyDeviceToHost, s),
                           "download"));
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "embedding_backward"));
    }
    for (int64_t t : tok) DLLM_REQUIRE(t >= 0 && static_cast<size_t>(t) < vocab, "token id out of range");
    // Stable counting sort by token (grad.hpp:433-447): groups in token order, positions ascending inside each.
    std::vector<int64_t> order(rows), starts, out_rows;
    std::vector<size_t> idx(rows);
    for (size_t r = 0; r < rows; ++r) idx[r] = r;
    std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) { return tok[a] < tok[b]; });
    for (size_t i = 0; i < rows; ++i) {
        order[i] = static_cast<int64_t>(idx[i]);
        if (i == 0 || tok[idx[i]] != tok[idx[i - 1]]) {
            starts.push_back(static_cast<int64_t>(i));
            out_rows.push_back(tok[idx[i]]);
        }
    }
    starts.push_back(static_cast<int64_t>(rows));
    Carve c(workspace, workspace_bytes);
    int64_t* d_order = c.take<int64_t>(rows);
    int64_t* d_start = c.take<int64_t>(rows + 1);
    int64_t* d_out = c.take<int64_t>(rows);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    const int64_t groups = static_cast<int64_t>(out_rows.size());
    DLLM_TRY(check_hip(hipMemsetAsync(out, 0, vocab * dim * sizeof(float), s), "memset"));
    if (groups > 0) {
        DLLM_TRY(check_hip(hipMemcpyAsync(d_order, order.data(), rows * sizeof(int64_t), hipMemcpyHostToDevice, s),
                           "upload"));
        DLLM_TRY(check_hip(hipMemcpyAsync(d_start, starts.data(), starts.size() * sizeof(int64_t),
                                          hipMemcpyHostToDevice, s), "upload"));
        DLLM_TRY(check_hip(hipMemcpyAsync(d_out, out_rows.data(), out_rows.size() * sizeof(int64_t),
                                          hipMemcpyHostToDevice, s), "upload"));
        DLLM_TRY(launch_embedding_groups(dy, static_cast<int64_t>(dim), d_order, d_start, d_out, groups, out,
                                         static_cast<int64_t>(dim), s));
    }
    // The host vectors are sources of asynchronous copies: wait before they go out of scope.
    return check_hip(hipStreamSynchronize(s), "embedding_backward");
}

size_t dllm_hip_sum_squares_workspace(size_t n) {
    const int64_t count = static_cast<int64_t>(n);
    const size_t blocks = exact_sum_squares_blocks(&count, 1);
    Layout l;
    l.add<int64_t>(2);           // first block, block count
    l.add<int64_t>(2 * blocks);  // block starts and counts
    l.add<char>(exact_sum_squares_workspace(blocks));
    l.add<double>(1);
    return l.bytes;
}

int dllm_hip_sum_squares(const float* values, size_t n, double* result, void* workspace, size_t workspace_bytes,
                         void* stream) {
    DLLM_REQUIRE(workspace_bytes >= dllm_hip_sum_squares_workspace(n), "workspace too small for sum_squares");
    const hipStream_t s = as_stream(stream);
    const int64_t count = static_cast<int64_t>(n), offset = 0;
    const size_t blocks = exact_sum_squares_blocks(&count, 1);
    std::vector<int64_t> tf(1), tb(1), bs(blocks), bc(blocks);
    exact_sum_squares_plan(&offset, &count, 1, tf.data(), tb.data(), bs.data(), bc.data());
    std::vector<int64_t> head = {tf[0], tb[0]}, table(bs);
    table.insert(table.end(), bc.begin(), bc.end());
    Carve c(workspace, workspace_bytes);
    int64_t* d_head = c.take<int64_t>(2);
    int64_t* d_table = c.take<int64_t>(2 * blocks);
    char* ws = c.take<char>(exact_sum_squares_workspace(blocks));
    double* d_result = c.take<double>(1);
    DLLM_REQUIRE(!c.overflow, "workspace layout overflow");
    DLLM_TRY(check_hip(hipMemcpyAsync(d_head, head.data(), 2 * sizeof(int64_t), hipMemcpyHostToDevice, s), "upload"));
    DLLM_TRY(check_hip(hipMemcpyAsync(d_table, table.data(), table.size() * sizeof(int64_t), hipMemcpyHostToDevice, s),
                       "upload"));
    ExactSumPlan plan;
    plan.tensors = 1;
    plan.blocks = static_cast<int64_t>(blocks);
    plan.tfirst = d_head;
    plan.tblocks = d_head + 1;
    plan.bstart = d_table;
    plan.bcount = d_table + blocks;
    DLLM_TRY(launch_exact_sum_squares(values, plan, ws, d_result, s));
    double host = 0.0;
    DLLM_TRY(check_hip(hipMemcpyAsync(&host, d_result, sizeof host, hipMemcpyDeviceToHost, s), "download"));
    DLLM_TRY(check_hip(hipStreamSynchronize(s), "sum_squares"));
    if (result) *result = host;
    return kOk;
}

int dllm_hip_adamw_step(float* param, const float* grad, float* m, float* v, size_t n, double lr, double beta1,
                        double beta2, double eps, double weight_decay, double bc1, double bc2, double grad_scale,
                        void* stream) {
    AdamWArgs a{lr, beta1, beta2, eps, bc1, bc2, grad_scale};
    return launch_adamw_plain(param, grad, m, v, static_cast<int64_t>(n), weight_decay, a, as_stream(stream));
}

int dllm_hip_gelu_tanh_backward(const float* x, const float* dy, float* out, size_t n, void* stream) {
    return launch_gelu_tanh_backward(x, dy, out, static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_softcap_backward(const float* x, const float* dy, float* out, size_t n, double cap, void* stream) {
    DLLM_REQUIRE(cap > 0.0, "cap must be positive");
    return launch_softcap_backward(x, dy, out, static_cast<int64_t>(n), cap, as_stream(stream));
}

int dllm_hip_softmax(const float* logits, float* out, size_t rows, size_t n, void* stream) {
    return launch_softmax_rows(logits, out, static_cast<int64_t>(rows), static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_column_mean(const float* x, float* out, size_t rows, size_t cols, void* stream) {
    return launch_column_mean(x, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), as_stream(stream));
}

size_t dllm_hip_dot_workspace(void) { return sizeof(float); }

int dllm_hip_dot(const float* a, const float* b, size_t n, float* result, void* workspace, size_t workspace_bytes,
                 void* stream) {
    DLLM_REQUIRE(result && workspace && workspace_bytes >= sizeof(float), "dot needs a result and a workspace");
    const hipStream_t s = as_stream(stream);
    float* d = static_cast<float*>(workspace);
    DLLM_TRY(launch_dot(a, b, static_cast<int64_t>(n), d, s));
    DLLM_TRY(check_hip(hipMemcpyAsync(result, d, sizeof(float), hipMemcpyDeviceToHost, s), "download"));
    return check_hip(hipStreamSynchronize(s), "dot");
}

int dllm_hip_moe_route(const float* logits, int64_t* indices, float* weights, size_t rows, size_t experts, size_t k,
                       int normalize, void* stream) {
    return launch_moe_route(logits, static_cast<int64_t>(rows), static_cast<int64_t>(experts),
                            static_cast<int64_t>(k), normalize, indices, weights, nullptr, as_stream(stream));
}

int dllm_hip_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights,
                                const float* dprobabilities, float* dlogits, size_t rows, size_t experts, size_t k,
                                int normalize, void* stream) {
    return launch_moe_route_backward(logits, indices, dweights, dprobabilities, static_cast<int64_t>(rows),
                                     static_cast<int64_t>(experts), static_cast<int64_t>(k), normalize, dlogits,
                                     as_stream(stream));
}

int dllm_hip_quantize_q8_0(const float* x, int8_t* q, float* scales, size_t n, void* stream) {
    DLLM_REQUIRE(n % 32 == 0, "q8_0 needs a weight whose in_features is a multiple of 32");
    return launch_quantize_q8_0(x, q, scales, static_cast<int64_t>(n), as_stream(stream));
}

int dllm_hip_dequantize_q8_0(const int8_t* q, const float* scales, float* out, size_t n, void* stream) {
    DLLM_REQUIRE(n % 32 == 0, "q8_0 needs a weight whose in_features is a multiple of 32");
    return launch_dequantize_q8_0(q, scales, out, static_cast<int64_t>(n), as_stream(stream));
}

size_t dllm_hip_lora_merge_workspace(size_t out_f, size_t in_f, size_t rank) {
    return lora_merge_workspace(static_cast<int64_t>(out_f), static_cast<int64_t>(in_f), static_cast<int64_t>(rank));
}

int dllm_hip_lora_merge(const float* weight, const float* a, const float* b, float* out, size_t out_f, size_t in_f,
                        size_t rank, double scale, void* workspace, size_t workspace_bytes, void* stream) {
    return launch_lora_merge(weight, a, b, out, static_cast<int64_t>(out_f), static_cast<int64_t>(in_f),
                             static_cast<int64_t>(rank), static_cast<float>(scale), workspace, workspace_bytes,
                             as_stream(stream));
}

size_t dllm_hip_lora_adapter_gradients_workspace(size_t out_f, size_t in_f, size_t rank) {
    return lora_adapter_gradients_workspace(static_cast<int64_t>(out_f), static_cast<int64_t>(in_f),
                                            static_cast<int64_t>(rank));
}

int dllm_hip_lora_adapter_gradients(const float* grad, const float* a, const float* b, float* da, float* db,
                                    size_t out_f, size_t in_f, size_t rank, double scale, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    return launch_lora_adapter_gradients(grad, a, b, da, db, static_cast<int64_t>(out_f), static_cast<int64_t>(in_f),
                                         static_cast<int64_t>(rank), static_cast<float>(scale), workspace,
                                         workspace_bytes, as_stream(stream));
}

}  // extern "C"
