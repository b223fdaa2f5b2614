// C shim over the reference's own header-only CPU kernels (cpp/include/dllm/*.hpp, compiled from the reference
// checkout by oracle/Makefile into oracle/_ref/libdllm_ref.so). TEST INFRASTRUCTURE ONLY: it pins the oracle's C
// restatement bit for bit and, driven by the oracle's step orchestration, times the reference CPU path as the
// baseline. The wrappers only adapt calling conventions; every computation is the reference's.
#include "dllm/fpenv.hpp"
#include "dllm/grad.hpp"
#include "dllm/interp.hpp"
#include "dllm/math.hpp"
#include "dllm/nn.hpp"
#include "dllm/parallel.hpp"
#include "dllm/quant.hpp"
#include "dllm/random.hpp"

#include <cstring>
#include <exception>
#include <vector>

#include "oracle.h"

namespace {

using dllm::FpEnvGuard;

void linear(const float* x, const float* w, const float* b, float* out, size_t rows, size_t in, size_t n) {
    FpEnvGuard guard;
    dllm::linear(x, w, b, out, rows, in, n);
}
void linear_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db, size_t rows,
                     size_t in, size_t n) {
    FpEnvGuard guard;
    dllm::linear_backward(x, w, dy, dx, dw, db, rows, in, n);
}
void rms_norm(const float* x, const float* w, float* out, size_t rows, size_t dim, double eps, int unit) {
    FpEnvGuard guard;
    dllm::rms_norm(x, w, out, rows, dim, eps, unit != 0);
}
void rms_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, size_t rows, size_t dim,
                       double eps, int unit) {
    FpEnvGuard guard;
    dllm::rms_norm_backward(x, w, dy, dx, dw, rows, dim, eps, unit != 0);
}
void rope(const float* x, const int64_t* pos, const double* f, float* out, size_t tokens, size_t heads, size_t hd,
          size_t rot, int interleaved, int inverse) {
    FpEnvGuard guard;
    dllm::rope(x, pos, f, out, tokens, heads, hd, rot, interleaved != 0, inverse != 0);
}
void attention(const float* q, const float* k, const float* v, float* out, size_t ql, size_t kl, size_t qh, size_t kh,
               size_t hd, size_t vd, double scale, int causal, size_t qo, size_t window, double softcap) {
    FpEnvGuard guard;
    dllm::attention(q, k, v, out, ql, kl, qh, kh, hd, vd, scale, causal != 0, qo, window, softcap);
}
void attention_backward(const float* q, const float* k, const float* v, const float* d, float* dq, float* dk,
                        float* dv, size_t ql, size_t kl, size_t qh, size_t kh, size_t hd, size_t vd, double scale,
                        int causal, size_t qo, size_t window, double softcap) {
    FpEnvGuard guard;
    dllm::attention_backward(q, k, v, d, dq, dk, dv, ql, kl, qh, kh, hd, vd, scale, causal != 0, qo, window, softcap);
}
void silu(const float* x, float* out, size_t n) {
    FpEnvGuard guard;
    dllm::parallel_elementwise(n, [&](std::size_t i) { out[i] = dllm::silu(x[i]); });
}
void swiglu(const float* g, const float* u, float* out, size_t n) {
    FpEnvGuard guard;
    dllm::gated_activation<dllm::silu>(g, u, out, n);
}
void silu_backward(const float* x, const float* dy, float* out, size_t n) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::silu_backward(x[i], dy[i]);
}
double cross_entropy(const float* l, const int64_t* t, float* dl, size_t rows, size_t vocab, double scale) {
    FpEnvGuard guard;
    try {
        return dllm::cross_entropy(l, t, dl, rows, vocab, scale);
    } catch (const std::exception&) {
        return __builtin_nan("");
    }
}
int embedding_backward(const float* dy, const int64_t* tokens, float* out, size_t rows, size_t dim, size_t vocab) {
    FpEnvGuard guard;
    try {
        dllm::embedding_backward(dy, tokens, out, rows, dim, vocab);
    } catch (const std::exception&) {
        return -1;
    }
    return 0;
}
double sum_squares(const float* v, size_t n) {
    FpEnvGuard guard;
    return dllm::sum_squares(v, n);
}
void adamw_step(float* p, const float* g, float* m, float* v, size_t n, double lr, double b1, double b2, double eps,
                double wd, double bc1, double bc2, double gs) {
    FpEnvGuard guard;
    dllm::adamw_step(p, g, m, v, n, lr, b1, b2, eps, wd, bc1, bc2, gs);
}
void softmax(const float* l, float* out, size_t n) {
    FpEnvGuard guard;
    std::vector<double> scratch(n);
    dllm::softmax(l, out, scratch.data(), n);
}
void moe_route(const float* l, int64_t* idx, float* w, size_t rows, size_t e, size_t k, int normalize) {
    FpEnvGuard guard;
    dllm::moe_route(l, idx, w, rows, e, k, normalize != 0);
}
void moe_route_backward(const float* l, const int64_t* idx, const float* dw, const float* dp, float* dl, size_t rows,
                        size_t e, size_t k, int normalize) {
    FpEnvGuard guard;
    dllm::moe_route_backward(l, idx, dw, dp, dl, rows, e, k, normalize != 0);
}
void column_mean(const float* x, float* out, size_t rows, size_t cols) {
    FpEnvGuard guard;
    dllm::column_mean(x, out, rows, cols);
}
float dot(const float* a, const float* b, size_t n) {
    FpEnvGuard guard;
    return dllm::dot(a, b, n);
}

void gelu_tanh(const float* x, float* out, size_t n) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::gelu_tanh(x[i]);
}
void gelu_tanh_backward(const float* x, const float* dy, float* out, size_t n) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::gelu_tanh_backward(x[i], dy[i]);
}
void softcap(const float* x, float* out, size_t n, double cap) {
    FpEnvGuard guard;
    dllm::softcap(x, out, n, cap);
}
void softcap_backward(const float* x, const float* dy, float* out, size_t n, double cap) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::softcap_backward(x[i], dy[i], cap);
}

const orc_ops kRefOps = {
    linear, linear_backward, rms_norm, rms_norm_backward, rope, attention, attention_backward, silu, swiglu,
    silu_backward, cross_entropy, embedding_backward, sum_squares, adamw_step, softmax, moe_route,
    moe_route_backward, column_mean, dot, gelu_tanh, gelu_tanh_backward, softcap, softcap_backward,
};

}  // namespace

extern "C" {

const orc_ops* ref_ops(void) { return &kRefOps; }

void ref_set_threads(size_t n) { dllm::ThreadPool::global().set_threads(n); }
size_t ref_threads(void) { return dllm::ThreadPool::global().threads(); }

double ref_exp(double x) { FpEnvGuard g; return dllm::exp(x); }
double ref_log(double x) { FpEnvGuard g; return dllm::log(x); }
double ref_sin(double x) { FpEnvGuard g; return dllm::sin(x); }
double ref_cos(double x) { FpEnvGuard g; return dllm::cos(x); }
double ref_tanh(double x) { FpEnvGuard g; return dllm::tanh(x); }
double ref_sigmoid(double x) { FpEnvGuard g; return dllm::sigmoid(x); }
float ref_silu(float x) { FpEnvGuard g; return dllm::silu(x); }
float ref_silu_backward(float x, float dy) { FpEnvGuard g; return dllm::silu_backward(x, dy); }
float ref_gelu_tanh(float x) { FpEnvGuard g; return dllm::gelu_tanh(x); }
float ref_gelu_tanh_backward(float x, float dy) { FpEnvGuard g; return dllm::gelu_tanh_backward(x, dy); }
float ref_softcap_backward(float x, float dy, double cap) { FpEnvGuard g; return dllm::softcap_backward(x, dy, cap); }

void ref_fill_gaussian(uint64_t seed, float* out, size_t n) {
    dllm::Random r(seed);
    for (size_t i = 0; i < n; ++i) out[i] = r.next_gaussian();
}
uint64_t ref_random_first(uint64_t seed) {
    dllm::Random r(seed);
    return r.next_u64();
}
void ref_linear_reference(const float* x, const float* w, const float* b, float* out, size_t rows, size_t in,
                          size_t n) {
    FpEnvGuard guard;
    dllm::linear_reference(x, w, b, out, rows, in, n);
}
void ref_attention_reference(const float* q, const float* k, const float* v, float* out, size_t ql, size_t kl,
                             size_t qh, size_t kh, size_t hd, size_t vd, double scale, int causal, size_t qo,
                             size_t window, double softcap) {
    FpEnvGuard guard;
    dllm::attention_reference(q, k, v, out, ql, kl, qh, kh, hd, vd, scale, causal != 0, qo, window, softcap);
}
void ref_quantize_q8_0(const float* x, int8_t* q, float* scales, size_t n) {
    FpEnvGuard guard;
    dllm::quantize_q8_0(x, q, scales, n);
}
void ref_linear_q8(const float* x, const int8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out) {
    FpEnvGuard guard;
    dllm::linear_q8(x, wq, ws, bias, out, rows, in, n_out);
}
void ref_quantize_q4_0(const float* x, uint8_t* packed, float* scales, size_t n) {
    FpEnvGuard guard;
    dllm::quantize_q4_0(x, packed, scales, n);
}
void ref_unpack_q4_0(const uint8_t* packed, int8_t* values, size_t n) { dllm::unpack_q4_0(packed, values, n); }
void ref_linear_q4(const float* x, const uint8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out) {
    FpEnvGuard guard;
    dllm::linear_q4(x, wq, ws, bias, out, rows, in, n_out);
}

double ref_erf(double x) { return dllm::erf(x); }
double ref_erfc(double x) { return dllm::erfc(x); }
void ref_gelu_n(const float* x, float* out, size_t n) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::gelu(x[i]);
}
void ref_gelu_backward_n(const float* x, const float* dy, float* out, size_t n) {
    FpEnvGuard guard;
    for (size_t i = 0; i < n; ++i) out[i] = dllm::gelu_backward(x[i], dy[i]);
}
void ref_layer_norm(const float* x, const float* w, const float* b, float* out, size_t rows, size_t dim, double eps) {
    FpEnvGuard guard;
    dllm::layer_norm(x, w, b, out, rows, dim, eps);
}
void ref_layer_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                             size_t rows, size_t dim, double eps) {
    FpEnvGuard guard;
    dllm::layer_norm_backward(x, w, dy, dx, dw, db, rows, dim, eps);
}
void ref_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out, size_t ql,
                          size_t kl, size_t heads, size_t hd, size_t vd, double scale) {
    FpEnvGuard guard;
    dllm::biased_attention(q, k, v, bias, out, ql, kl, heads, hd, vd, scale);
}
void ref_biased_attention_weights(const float* q, const float* k, const float* bias, float* out, size_t ql, size_t kl,
                                  size_t heads, size_t hd, double scale) {
    dllm::biased_attention_weights(q, k, bias, out, ql, kl, heads, hd, scale);
}
void ref_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                   const float* dout, float* dq, float* dk, float* dv, float* dbias, size_t ql,
                                   size_t kl, size_t heads, size_t hd, size_t vd, double scale) {
    FpEnvGuard guard;
    dllm::biased_attention_backward(q, k, v, bias, dout, dq, dk, dv, dbias, ql, kl, heads, hd, vd, scale);
}

}  // extern "C"
