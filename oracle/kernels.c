/*
 * CPU oracle kernels (TEST INFRASTRUCTURE ONLY; see oracle.h). Plain C restatement of the reference's kernels, one
 * scalar loop per output, in the exact evaluation order of the cited reference lines. Single-threaded on purpose:
 * the oracle states the order, it does not race the GPU.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* 2^k as a double built from its bits (math.hpp:55-60). */
static double pow2i(int k) {
    const uint64_t bits = (uint64_t)(k + 1023) << 52;
    double r;
    memcpy(&r, &bits, sizeof r);
    return r;
}

/* n! for small n, exact in double. */
static double factorial(int n) {
    double f = 1.0;
    for (int i = 2; i <= n; ++i) f *= (double)i;
    return f;
}

/* e^x (math.hpp:64-109): x = k ln2 + r with a two-part ln2, the degree-13 Taylor polynomial of e^r in Horner form
 * from the 1/13! term down, then 2^k applied in steps that keep every factor a normal double. */
double orc_exp(double x) {
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double inv_ln2 = 1.44269504088896338700e+00;
    if (x != x) return x;
    if (x > 709.78) return INFINITY;
    if (x < -745.2) return 0.0;
    const double kd = x * inv_ln2;
    const int k = (int)(kd >= 0 ? kd + 0.5 : kd - 0.5);
    const double r = (x - k * ln2_hi) - k * ln2_lo;
    double p = 1.0 / factorial(13);
    for (int n = 12; n >= 0; --n) p = p * r + 1.0 / factorial(n);
    int e = k;
    while (e > 1023) { p *= pow2i(1023); e -= 1023; }
    while (e < -1022) { p *= pow2i(-1022); e += 1022; }
    return p * pow2i(e);
}

/* log x (math.hpp:113-162): x = m 2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s), s = (m-1)/(m+1), odd series
 * with the 1/25 .. 1/3 coefficients in Horner form in s^2, then e ln2 with the two-part ln2. */
double orc_log(double x) {
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double sqrt_half = 7.07106781186547524401e-01;
    if (x != x || x < 0.0) return NAN;
    if (x == 0.0) return -INFINITY;
    if (x == INFINITY) return x;
    int e = 0;
    if (x < DBL_MIN) { x *= pow2i(54); e -= 54; }
    uint64_t bits;
    memcpy(&bits, &x, sizeof bits);
    e += (int)((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL;
    double m;
    memcpy(&m, &bits, sizeof m);
    if (m >= 2.0 * sqrt_half) { m *= 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 25.0;
    for (int d = 23; d >= 3; d -= 2) p = p * s2 + 1.0 / (double)d;
    const double log_m = 2.0 * s + 2.0 * s * s2 * p;
    return (e * ln2_hi + log_m) + e * ln2_lo;
}

/* Taylor kernels on [-pi/4, pi/4] (math.hpp:168-190): alternating 1/n! coefficients, Horner in r^2. */
static double sin_kernel(double r) {
    const double r2 = r * r;
    double p = -1.0 / factorial(15);
    for (int n = 13; n >= 3; n -= 2) {
        const double c = 1.0 / factorial(n);
        p = ((n / 2) % 2 == 0) ? p * r2 + c : p * r2 - c;
    }
    return r + r * r2 * p;
}

static double cos_kernel(double r) {
    const double r2 = r * r;
    double p = 1.0 / factorial(16);
    for (int n = 14; n >= 4; n -= 2) {
        const double c = 1.0 / factorial(n);
        p = ((n / 2) % 2 == 0) ? p * r2 + c : p * r2 - c;
    }
    return (1.0 - 0.5 * r2) + r2 * r2 * p;
}

/* Cody-Waite reduction by pi/2 with fdlibm's three 33-bit parts (math.hpp:194-216). */
static double reduce_half_pi(double x, int* quadrant) {
    const double two_over_pi = 6.36619772367581382433e-01;
    const double pio2_1 = 1.57079632673412561417e+00;
    const double pio2_2 = 6.07710050630396597660e-11;
    const double pio2_3 = 2.02226624871116645580e-21;
    const double pio2_3t = 8.47842766036889956997e-32;
    const double two_52 = 4503599627370496.0;
    const double two_62 = 4611686018427387904.0;
    const double nd = x * two_over_pi;
    double n = nd;
    if (nd < two_52 && nd > -two_52) {
        n = nd >= 0 ? (double)(long long)(nd + 0.5) : (double)(long long)(nd - 0.5);
    }
    const double r = (((x - n * pio2_1) - n * pio2_2) - n * pio2_3) - n * pio2_3t;
    *quadrant = (n < two_62 && n > -two_62) ? (int)((long long)n & 3) : 0;
    return r;
}

double orc_sin(double x) {
    if (x != x || x == INFINITY || x == -INFINITY) return NAN;
    int q;
    const double r = reduce_half_pi(x, &q);
    switch (q) {
        case 0: return sin_kernel(r);
        case 1: return cos_kernel(r);
        case 2: return -sin_kernel(r);
        default: return -cos_kernel(r);
    }
}

double orc_cos(double x) {
    if (x != x || x == INFINITY || x == -INFINITY) return NAN;
    int q;
    const double r = reduce_half_pi(x, &q);
    switch (q) {
        case 0: return cos_kernel(r);
        case 1: return -sin_kernel(r);
        case 2: return -cos_kernel(r);
        default: return sin_kernel(r);
    }
}

/* tanh (math.hpp:296-319): odd Taylor series below 0.125, 1 beyond 22, else 1 - 2 / (e^(2a) + 1). */
double orc_tanh(double x) {
    if (x != x) return x;
    const double a = x < 0 ? -x : x;
    double t;
    if (a < 0.125) {
        const double a2 = a * a;
        double p = -929569.0 / 638512875.0;
        p = p * a2 + 21844.0 / 6081075.0;
        p = p * a2 - 1382.0 / 155925.0;
        p = p * a2 + 62.0 / 2835.0;
        p = p * a2 - 17.0 / 315.0;
        p = p * a2 + 2.0 / 15.0;
        p = p * a2 - 1.0 / 3.0;
        t = a + a * a2 * p;
    } else if (a > 22.0) {
        t = 1.0;
    } else {
        t = 1.0 - 2.0 / (orc_exp(2.0 * a) + 1.0);
    }
    return x < 0 ? -t : t;
}

double orc_sigmoid(double x) {
    if (x >= 0) return 1.0 / (1.0 + orc_exp(-x));
    const double e = orc_exp(x);
    return e / (1.0 + e);
}

float orc_dot(const float* a, const float* b, size_t n) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += (double)a[i] * (double)b[i];
    return (float)acc;
}

size_t orc_argmax(const float* v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

void orc_softmax(const float* logits, float* out, size_t n) {
    double* e = (double*)malloc(n * sizeof(double));
    const double max = logits[orc_argmax(logits, n)];
    double total = 0.0;
    for (size_t i = 0; i < n; ++i) {
        e[i] = orc_exp((double)logits[i] - max);
        total += e[i];
    }
    const double inv = 1.0 / total;
    for (size_t i = 0; i < n; ++i) out[i] = (float)(e[i] * inv);
    free(e);
}

/* ---- xoshiro256** seeded by SplitMix64 (random.hpp:10-55) ---- */
static uint64_t splitmix(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void orc_random_init(orc_random* r, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) r->s[i] = splitmix(&sm);
}

uint64_t orc_random_next(orc_random* r) {
    uint64_t* s = r->s;
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

double orc_random_double(orc_random* r) { return (double)(orc_random_next(r) >> 11) * (1.0 / 9007199254740992.0); }

float orc_random_gaussian(orc_random* r) {
    double sum = 0.0;
    for (int i = 0; i < 12; ++i) sum += orc_random_double(r);
    return (float)(sum - 6.0);
}

void orc_fill_gaussian(uint64_t seed, float* out, size_t n) {
    orc_random r;
    orc_random_init(&r, seed);
    for (size_t i = 0; i < n; ++i) out[i] = orc_random_gaussian(&r);
}

/* ---- forward kernels ---- */

/* linear_reference (nn.hpp:28-50): out[r, n] = f32(sum_k x[r, k] w[n, k] (+ bias[n])), k ascending in double, the
 * bias added to the double sum. */
void orc_linear(const float* x, const float* w, const float* bias, float* out, size_t rows, size_t in,
                size_t out_features) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * in;
        for (size_t n = 0; n < out_features; ++n) {
            const float* wn = w + n * in;
            double acc = 0.0;
            for (size_t k = 0; k < in; ++k) acc += (double)xr[k] * (double)wn[k];
            if (bias) acc += bias[n];
            out[r * out_features + n] = (float)acc;
        }
    }
}

/* rms_norm (nn.hpp:391-408): inv = 1 / sqrt(sum x^2 / dim + eps); out = f32((x inv) scale). */
void orc_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t dim, double eps, int unit_offset) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        double sum_sq = 0.0;
        for (size_t i = 0; i < dim; ++i) sum_sq += (double)xr[i] * (double)xr[i];
        const double inv = 1.0 / sqrt(sum_sq / (double)dim + eps);
        for (size_t i = 0; i < dim; ++i) {
            double scale = 1.0;
            if (w) scale = unit_offset ? 1.0 + (double)w[i] : (double)w[i];
            out[r * dim + i] = (float)((double)xr[i] * inv * scale);
        }
    }
}

float orc_silu(float x) {
    const double d = x;
    return (float)(d * orc_sigmoid(d));
}

/* gated_activation<silu> (nn.hpp:489-492): the activation rounded to float, then a float multiply. */
void orc_swiglu(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_silu(gate[i]) * up[i];
}

/* rope (nn.hpp:501-530): angle = pos * inv_freq[i] in double; pairs (i, i + half) or (2i, 2i + 1). */
void orc_rope(const float* x, const int64_t* positions, const double* inv_freq, float* out, size_t tokens,
              size_t heads, size_t head_dim, size_t rotary_dim, int interleaved, int inverse) {
    const size_t half = rotary_dim / 2;
    double* ct = (double*)malloc((half ? half : 1) * sizeof(double));
    double* st = (double*)malloc((half ? half : 1) * sizeof(double));
    for (size_t t = 0; t < tokens; ++t) {
        const double pos = (double)positions[t];
        for (size_t i = 0; i < half; ++i) {
            const double angle = pos * inv_freq[i];
            ct[i] = orc_cos(angle);
            st[i] = inverse ? -orc_sin(angle) : orc_sin(angle);
        }
        for (size_t h = 0; h < heads; ++h) {
            const float* xh = x + (t * heads + h) * head_dim;
            float* oh = out + (t * heads + h) * head_dim;
            for (size_t i = 0; i < half; ++i) {
                const size_t i0 = interleaved ? 2 * i : i;
                const size_t i1 = interleaved ? 2 * i + 1 : i + half;
                const double a = xh[i0];
                const double b = xh[i1];
                oh[i0] = (float)(a * ct[i] - b * st[i]);
                oh[i1] = (float)(a * st[i] + b * ct[i]);
            }
            for (size_t i = rotary_dim; i < head_dim; ++i) oh[i] = xh[i];
        }
    }
    free(ct);
    free(st);
}

/* attention_span (nn.hpp:733-748): the keys query t sees. */
static void span_of(size_t t, size_t kv_len, int causal, size_t q_offset, size_t window, size_t* first,
                    size_t* count) {
    const size_t pos = q_offset + t;
    if (!causal) {
        if (window == 0) { *first = 0; *count = kv_len; return; }
        const size_t f = pos + 1 > window ? pos + 1 - window : 0;
        const size_t last = pos + window < kv_len ? pos + window : kv_len;
        *first = f;
        *count = last > f ? last - f : 0;
        return;
    }
    const size_t end = pos + 1 < kv_len ? pos + 1 : kv_len;
    const size_t f = window != 0 && end > window ? end - window : 0;
    *first = f;
    *count = end - f;
}

/* attention_reference / attention_row / attention_finish (nn.hpp:535-615, 799-823): per (query, head) row, scores
 * dot (head_dim ascending) times scale, optional soft-cap, max, exponentials and their total over keys ascending,
 * value sums of the unnormalised weights over keys ascending, times 1/total once. */
void orc_attention(const float* q, const float* k, const float* v, float* out, size_t q_len, size_t kv_len,
                   size_t q_heads, size_t kv_heads, size_t head_dim, size_t value_dim, double scale, int causal,
                   size_t q_offset, size_t window, double softcap) {
    const size_t group = q_heads / kv_heads;
    double* s = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* acc = (double*)malloc((value_dim ? value_dim : 1) * sizeof(double));
    for (size_t t = 0; t < q_len; ++t) {
        size_t first, count;
        span_of(t, kv_len, causal, q_offset, window, &first, &count);
        for (size_t h = 0; h < q_heads; ++h) {
            const size_t g = h / group;
            const float* qh = q + (t * q_heads + h) * head_dim;
            float* oh = out + (t * q_heads + h) * value_dim;
            if (count == 0) {
                for (size_t i = 0; i < value_dim; ++i) oh[i] = 0.0f;
                continue;
            }
            for (size_t j = 0; j < count; ++j) {
                const float* kj = k + ((first + j) * kv_heads + g) * head_dim;
                double d = 0.0;
                for (size_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
                s[j] = d * scale;
            }
            if (softcap > 0.0)
                for (size_t j = 0; j < count; ++j) s[j] = softcap * orc_tanh(s[j] / softcap);
            double max = s[0];
            for (size_t j = 1; j < count; ++j)
                if (s[j] > max) max = s[j];
            double total = 0.0;
            for (size_t j = 0; j < count; ++j) {
                s[j] = orc_exp(s[j] - max);
                total += s[j];
            }
            for (size_t i = 0; i < value_dim; ++i) acc[i] = 0.0;
            for (size_t j = 0; j < count; ++j) {
                const float* vj = v + ((first + j) * kv_heads + g) * value_dim;
                for (size_t i = 0; i < value_dim; ++i) acc[i] += s[j] * (double)vj[i];
            }
            const double inv = 1.0 / total;
            for (size_t i = 0; i < value_dim; ++i) oh[i] = (float)(acc[i] * inv);
        }
    }
    free(s);
    free(acc);
}

/* moe_route (nn.hpp:864-896): softmax, top-k in a total order (larger first, ties to the lower expert), optional
 * renormalisation by the chosen total summed in double in rank order. */
void orc_moe_route(const float* logits, int64_t* indices, float* weights, size_t rows, size_t experts, size_t k,
                   int normalize) {
    float* p = (float*)malloc(experts * sizeof(float));
    unsigned char* taken = (unsigned char*)malloc(experts);
    for (size_t r = 0; r < rows; ++r) {
        orc_softmax(logits + r * experts, p, experts);
        memset(taken, 0, experts);
        double total = 0.0;
        for (size_t j = 0; j < k; ++j) {
            size_t best = experts;
            for (size_t e = 0; e < experts; ++e)
                if (!taken[e] && (best == experts || p[e] > p[best])) best = e;
            taken[best] = 1;
            indices[r * k + j] = (int64_t)best;
            weights[r * k + j] = p[best];
            total += (double)p[best];
        }
        if (normalize)
            for (size_t j = 0; j < k; ++j) weights[r * k + j] = (float)((double)weights[r * k + j] / total);
    }
    free(p);
    free(taken);
}

/* ---- backward kernels ---- */

/* linear_backward (grad.hpp:26-72). */
void orc_linear_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                         size_t rows, size_t in, size_t out_features) {
    double* acc = (double*)malloc((in ? in : 1) * sizeof(double));
    if (dx) {
        for (size_t r = 0; r < rows; ++r) {
            for (size_t k = 0; k < in; ++k) acc[k] = 0.0;
            for (size_t n = 0; n < out_features; ++n) {
                const double g = dy[r * out_features + n];
                const float* wn = w + n * in;
                for (size_t k = 0; k < in; ++k) acc[k] += g * (double)wn[k];
            }
            for (size_t k = 0; k < in; ++k) dx[r * in + k] = (float)acc[k];
        }
    }
    if (dw || db) {
        for (size_t n = 0; n < out_features; ++n) {
            for (size_t k = 0; k < in; ++k) acc[k] = 0.0;
            double bias_acc = 0.0;
            for (size_t r = 0; r < rows; ++r) {
                const double g = dy[r * out_features + n];
                bias_acc += g;
                if (dw) {
                    const float* xr = x + r * in;
                    for (size_t k = 0; k < in; ++k) acc[k] += g * (double)xr[k];
                }
            }
            if (dw)
                for (size_t k = 0; k < in; ++k) dw[n * in + k] = (float)acc[k];
            if (db) db[n] = (float)bias_acc;
        }
    }
    free(acc);
}

/* rms_norm_backward (grad.hpp:79-111). The (g dy) x and (dy x) inv products round, so no fused multiply-add. */
void orc_rms_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, size_t rows,
                           size_t dim, double eps, int unit_offset) {
    const double offset = unit_offset ? 1.0 : 0.0;
    double* dw_acc = (double*)calloc(dim ? dim : 1, sizeof(double));
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        const float* dyr = dy + r * dim;
        double sum_sq = 0.0;
        for (size_t i = 0; i < dim; ++i) sum_sq += (double)xr[i] * (double)xr[i];
        const double inv = 1.0 / sqrt(sum_sq / (double)dim + eps);
        double dot_acc = 0.0;
        for (size_t i = 0; i < dim; ++i) {
            const double wi = w ? offset + (double)w[i] : 1.0;
            dot_acc += wi * (double)dyr[i] * (double)xr[i];
            dw_acc[i] += (double)dyr[i] * (double)xr[i] * inv;
        }
        const double coef = dot_acc * inv * inv * inv / (double)dim;
        if (dx) {
            for (size_t i = 0; i < dim; ++i) {
                const double wi = w ? offset + (double)w[i] : 1.0;
                dx[r * dim + i] = (float)(inv * wi * (double)dyr[i] - (double)xr[i] * coef);
            }
        }
    }
    if (dw)
        for (size_t i = 0; i < dim; ++i) dw[i] = (float)dw_acc[i];
    free(dw_acc);
}

/* silu_backward (grad.hpp:177-181): dy s (1 + x (1 - s)) in double, rounded once. */
float orc_silu_backward(float x, float dy) {
    const double d = x;
    const double s = orc_sigmoid(d);
    return (float)((double)dy * s * (1.0 + d * (1.0 - s)));
}

/* gelu_tanh (nn.hpp:481-485): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in double, rounded once. */
float orc_gelu_tanh(float x) {
    const double c = 7.97884560802865355879e-01; /* sqrt(2 / pi) */
    const double d = x;
    return (float)(0.5 * d * (1.0 + orc_tanh(c * (d + 0.044715 * d * d * d))));
}

/* gelu_tanh_backward (grad.hpp:183-191): u = sqrt(2/pi) (x + 0.044715 x^3), t = tanh(u), dy times
 * 0.5 (1 + t) + 0.5 x (1 - t^2) sqrt(2/pi) (1 + 3 0.044715 x^2), in double, rounded once. */
float orc_gelu_tanh_backward(float x, float dy) {
    const double c = 7.97884560802865355879e-01; /* sqrt(2 / pi) */
    const double d = x;
    const double t = orc_tanh(c * (d + 0.044715 * d * d * d));
    const double slope = 0.5 * (1.0 + t) + 0.5 * d * (1.0 - t * t) * c * (1.0 + 3.0 * 0.044715 * d * d);
    return (float)((double)dy * slope);
}

/* softcap_backward (grad.hpp:193-197): dy (1 - tanh(x / cap)^2), rounded once. */
float orc_softcap_backward(float x, float dy, double cap) {
    const double t = orc_tanh((double)x / cap);
    return (float)((double)dy * (1.0 - t * t));
}

/* attention_backward (grad.hpp:206-301): rows (t ascending, then h ascending) recompute p exactly, then dq per row and
 * the key/value gradients as double accumulators visited in (t, h) order. */
void orc_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                            float* dv, size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                            size_t head_dim, size_t value_dim, double scale, int causal, size_t q_offset,
                            size_t window, double softcap) {
    const size_t group = q_heads / kv_heads;
    double* probs = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* slopes = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* dprobs = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* dq_acc = (double*)malloc((head_dim ? head_dim : 1) * sizeof(double));
    double* dk_acc = (double*)calloc(kv_len * kv_heads * head_dim + 1, sizeof(double));
    double* dv_acc = (double*)calloc(kv_len * kv_heads * value_dim + 1, sizeof(double));
    for (size_t j = 0; j < kv_len; ++j) slopes[j] = 1.0;
    for (size_t t = 0; t < q_len; ++t) {
        size_t first, visible;
        span_of(t, kv_len, causal, q_offset, window, &first, &visible);
        const float* kw = k + first * kv_heads * head_dim;
        const float* vw = v + first * kv_heads * value_dim;
        double* dkw = dk_acc + first * kv_heads * head_dim;
        double* dvw = dv_acc + first * kv_heads * value_dim;
        for (size_t h = 0; h < q_heads; ++h) {
            const size_t g = h / group;
            const float* qh = q + (t * q_heads + h) * head_dim;
            const float* doh = dout + (t * q_heads + h) * value_dim;
            float* dqh = dq + (t * q_heads + h) * head_dim;
            if (visible == 0) {
                for (size_t i = 0; i < head_dim; ++i) dqh[i] = 0.0f;
                continue;
            }
            double max = 0.0;
            for (size_t j = 0; j < visible; ++j) {
                const float* kj = kw + (j * kv_heads + g) * head_dim;
                double d = 0.0;
                for (size_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
                probs[j] = d * scale;
                if (softcap > 0.0) {
                    const double th = orc_tanh(probs[j] / softcap);
                    probs[j] = softcap * th;
                    slopes[j] = 1.0 - th * th;
                }
                if (j == 0 || probs[j] > max) max = probs[j];
            }
            double total = 0.0;
            for (size_t j = 0; j < visible; ++j) {
                probs[j] = orc_exp(probs[j] - max);
                total += probs[j];
            }
            const double inv = 1.0 / total;
            double weighted = 0.0;
            for (size_t j = 0; j < visible; ++j) {
                probs[j] *= inv;
                const float* vj = vw + (j * kv_heads + g) * value_dim;
                double d = 0.0;
                for (size_t i = 0; i < value_dim; ++i) d += (double)doh[i] * (double)vj[i];
                dprobs[j] = d;
                weighted += probs[j] * d;
            }
            for (size_t i = 0; i < head_dim; ++i) dq_acc[i] = 0.0;
            for (size_t j = 0; j < visible; ++j) {
                const double ds = probs[j] * (dprobs[j] - weighted) * slopes[j] * scale;
                const float* kj = kw + (j * kv_heads + g) * head_dim;
                double* dkj = dkw + (j * kv_heads + g) * head_dim;
                double* dvj = dvw + (j * kv_heads + g) * value_dim;
                for (size_t i = 0; i < head_dim; ++i) {
                    dq_acc[i] += ds * (double)kj[i];
                    dkj[i] += ds * (double)qh[i];
                }
                for (size_t i = 0; i < value_dim; ++i) dvj[i] += probs[j] * (double)doh[i];
            }
            for (size_t i = 0; i < head_dim; ++i) dqh[i] = (float)dq_acc[i];
        }
    }
    for (size_t i = 0; i < kv_len * kv_heads * head_dim; ++i) dk[i] = (float)dk_acc[i];
    for (size_t i = 0; i < kv_len * kv_heads * value_dim; ++i) dv[i] = (float)dv_acc[i];
    free(probs); free(slopes); free(dprobs); free(dq_acc); free(dk_acc); free(dv_acc);
}

/* cross_entropy (grad.hpp:395-426). Returns NAN for a target out of range (the reference throws). */
double orc_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, size_t rows, size_t vocab,
                         double scale) {
    double* e = (double*)malloc((vocab ? vocab : 1) * sizeof(double));
    double loss = 0.0;
    for (size_t r = 0; r < rows; ++r) {
        const float* lr = logits + r * vocab;
        float* dr = dlogits + r * vocab;
        const int64_t target = targets[r];
        if (target < 0) {
            for (size_t j = 0; j < vocab; ++j) dr[j] = 0.0f;
            continue;
        }
        if ((size_t)target >= vocab) { free(e); return NAN; }
        const double max = lr[orc_argmax(lr, vocab)];
        double total = 0.0;
        for (size_t j = 0; j < vocab; ++j) {
            e[j] = orc_exp((double)lr[j] - max);
            total += e[j];
        }
        loss += max + orc_log(total) - (double)lr[target];
        const double inv = 1.0 / total;
        for (size_t j = 0; j < vocab; ++j) {
            const double onehot = (size_t)target == j ? 1.0 : 0.0;
            dr[j] = (float)((e[j] * inv - onehot) * scale);
        }
    }
    free(e);
    return loss;
}

/* embedding_backward (grad.hpp:431-464): rows grouped per token by a stable counting sort, summed in position order
 * in double. Returns -1 for a token out of range. */
int orc_embedding_backward(const float* dy, const int64_t* tokens, float* out, size_t rows, size_t dim,
                           size_t vocab) {
    for (size_t r = 0; r < rows; ++r)
        if (tokens[r] < 0 || (size_t)tokens[r] >= vocab) return -1;
    double* acc = (double*)malloc((dim ? dim : 1) * sizeof(double));
    for (size_t t = 0; t < vocab; ++t) {
        for (size_t i = 0; i < dim; ++i) acc[i] = 0.0;
        for (size_t r = 0; r < rows; ++r) {
            if ((size_t)tokens[r] != t) continue;
            for (size_t i = 0; i < dim; ++i) acc[i] += (double)dy[r * dim + i];
        }
        for (size_t i = 0; i < dim; ++i) out[t * dim + i] = (float)acc[i];
    }
    free(acc);
    return 0;
}

double orc_sum_squares(const float* v, size_t n) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += (double)v[i] * (double)v[i];
    return acc;
}

/* adamw_step (grad.hpp:481-495). */
void orc_adamw_step(float* param, const float* grad, float* m, float* v, size_t n, double lr, double beta1,
                    double beta2, double eps, double weight_decay, double bc1, double bc2, double grad_scale) {
    const double decay = 1.0 - lr * weight_decay;
    for (size_t i = 0; i < n; ++i) {
        const double g = (double)grad[i] * grad_scale;
        const float m_new = (float)(beta1 * (double)m[i] + (1.0 - beta1) * g);
        const float v_new = (float)(beta2 * (double)v[i] + (1.0 - beta2) * g * g);
        m[i] = m_new;
        v[i] = v_new;
        const double m_hat = (double)m_new / bc1;
        const double v_hat = (double)v_new / bc2;
        param[i] = (float)((double)param[i] * decay - lr * m_hat / (sqrt(v_hat) + eps));
    }
}

/* moe_route_backward (grad.hpp:507-541). */
void orc_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights,
                            const float* dprobabilities, float* dlogits, size_t rows, size_t experts, size_t k,
                            int normalize) {
    float* p = (float*)malloc(experts * sizeof(float));
    double* dp = (double*)malloc(experts * sizeof(double));
    for (size_t r = 0; r < rows; ++r) {
        orc_softmax(logits + r * experts, p, experts);
        for (size_t e = 0; e < experts; ++e) dp[e] = dprobabilities ? (double)dprobabilities[r * experts + e] : 0.0;
        double total = 0.0, weighted = 0.0;
        for (size_t j = 0; j < k; ++j) {
            const int64_t e = indices[r * k + j];
            total += (double)p[e];
            weighted += (double)dweights[r * k + j] * (double)p[e];
        }
        for (size_t j = 0; j < k; ++j) {
            const size_t e = (size_t)indices[r * k + j];
            const double dw = dweights[r * k + j];
            dp[e] += normalize ? dw / total - weighted / (total * total) : dw;
        }
        double dot = 0.0;
        for (size_t e = 0; e < experts; ++e) dot += (double)p[e] * dp[e];
        for (size_t e = 0; e < experts; ++e) dlogits[r * experts + e] = (float)((double)p[e] * (dp[e] - dot));
    }
    free(p);
    free(dp);
}

/* column_mean (interp.hpp:146-155). */
void orc_column_mean(const float* x, float* out, size_t rows, size_t cols) {
    for (size_t c = 0; c < cols; ++c) {
        double total = 0.0;
        for (size_t r = 0; r < rows; ++r) total += x[r * cols + c];
        out[c] = rows > 0 ? (float)(total / (double)rows) : 0.0f;
    }
}

/* round half to even of a float with exact operations (quant.hpp:27-38). */
static float round_half_even(float v) {
    const float f = floorf(v);
    const float diff = v - f;
    if (diff > 0.5f) return f + 1.0f;
    if (diff < 0.5f) return f;
    return fmodf(f, 2.0f) == 0.0f ? f : f + 1.0f;
}

/* quantize_q8_0 (quant.hpp:41-60): 32-value blocks, d = amax / 127, q = rne(x / d) clamped to +-127. */
void orc_quantize_q8_0(const float* x, int8_t* q, float* scales, size_t n) {
    for (size_t b = 0; b * 32 < n; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.0f;
        for (size_t i = 0; i < 32; ++i) {
            const float a = fabsf(xb[i]);
            if (a > amax && isfinite(a)) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        scales[b] = d;
        for (size_t i = 0; i < 32; ++i) {
            float val = isfinite(xb[i]) ? round_half_even(xb[i] * id) : 0.0f;
            val = val > 127.0f ? 127.0f : (val < -127.0f ? -127.0f : val);
            q[b * 32 + i] = (int8_t)val;
        }
    }
}

/* linear_q8 (quant.hpp:143-169, 355-383): each row's activations quantised to Q8_0 (quant.hpp:27-60), then per output
 * acc = sum over blocks b ascending of (f64(xs[r][b]) f64(ws[n][b])) f64(isum_b), isum_b the exact int32 dot of the
 * block's 32 int8 pairs; acc += bias[n]; rounded to float once. in_features is a multiple of 32. */
void orc_linear_q8(const float* x, const int8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out) {
    const size_t blocks = in / 32;
    int8_t* xq = (int8_t*)malloc(in > 0 ? in : 1);
    float* xs = (float*)malloc((blocks > 0 ? blocks : 1) * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        orc_quantize_q8_0(x + r * in, xq, xs, in);
        for (size_t n = 0; n < n_out; ++n) {
            double acc = 0.0;
            for (size_t b = 0; b < blocks; ++b) {
                int32_t isum = 0;
                for (size_t i = 0; i < 32; ++i) isum += (int32_t)xq[b * 32 + i] * (int32_t)wq[n * in + b * 32 + i];
                acc += ((double)xs[b] * (double)ws[n * blocks + b]) * (double)isum;
            }
            if (bias) acc += bias[n];
            out[r * n_out + n] = (float)acc;
        }
    }
    free(xq);
    free(xs);
}

/* quantize_q4_0 (quant.hpp:67-94): amax over finite values, d = amax / 7, q = round-half-even(x / d) clamped to +-7;
 * byte j of a block holds q_j + 8 (low four bits) and q_(j+16) + 8 (high four bits). */
void orc_quantize_q4_0(const float* x, uint8_t* packed, float* scales, size_t n) {
    for (size_t b = 0; b * 32 < n; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.0f;
        for (size_t i = 0; i < 32; ++i) {
            const float a = fabsf(xb[i]);
            if (a > amax && isfinite(a)) amax = a;
        }
        const float d = amax / 7.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        scales[b] = d;
        int q[32];
        for (size_t i = 0; i < 32; ++i) {
            float val = isfinite(xb[i]) ? round_half_even(xb[i] * id) : 0.0f;
            val = val > 7.0f ? 7.0f : (val < -7.0f ? -7.0f : val);
            q[i] = (int)val;
        }
        for (size_t j = 0; j < 16; ++j) packed[b * 16 + j] = (uint8_t)((q[j] + 8) | ((q[j + 16] + 8) << 4));
    }
}

/* unpack_q4_0 (quant.hpp:97-108). */
void orc_unpack_q4_0(const uint8_t* packed, int8_t* values, size_t n) {
    for (size_t b = 0; b * 32 < n; ++b)
        for (size_t j = 0; j < 16; ++j) {
            values[b * 32 + j] = (int8_t)((packed[b * 16 + j] & 0x0F) - 8);
            values[b * 32 + j + 16] = (int8_t)((packed[b * 16 + j] >> 4) - 8);
        }
}

/* linear_q4 (quant.hpp:385-403): the weights unpacked to int8, then exactly linear_q8. */
void orc_linear_q4(const float* x, const uint8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out) {
    int8_t* w = (int8_t*)malloc(n_out * in > 0 ? n_out * in : 1);
    orc_unpack_q4_0(wq, w, n_out * in);
    orc_linear_q8(x, w, ws, bias, out, rows, in, n_out);
    free(w);
}

/* ---- encoder and T5 training kernels (grad.hpp:112-174, 300-389; nn.hpp:412-432, 474-478, 827-856) ---- */

/* erfc(a) for a >= 2.5 (math.hpp:332-341): e^(-a^2) / sqrt(pi) / K(a), K the Laplace continued fraction evaluated
 * backwards from depth 80. */
static double erfc_tail(double a) {
    const double inv_sqrt_pi = 5.64189583547756286948e-01;
    double k = a;
    for (int n = 80; n >= 1; --n) k = a + (0.5 * n) / k;
    return orc_exp(-a * a) * inv_sqrt_pi / k;
}

/* erf (math.hpp:345-370): the 60-term Maclaurin series below 2.5, 1 - erfc_tail(|x|) up to 6, 1 beyond. */
double orc_erf(double x) {
    const double two_over_sqrt_pi = 1.12837916709551257390e+00;
    if (x != x) return x;
    const double a = x < 0 ? -x : x;
    double result;
    if (a < 2.5) {
        const double a2 = a * a;
        double term = a, total = a;
        for (int n = 1; n < 60; ++n) {
            term = -term * a2 / n;
            total += term / (2 * n + 1);
        }
        result = two_over_sqrt_pi * total;
    } else if (a > 6.0) {
        result = 1.0;
    } else {
        result = 1.0 - erfc_tail(a);
    }
    return x < 0 ? -result : result;
}

/* erfc (math.hpp:373-384). */
double orc_erfc(double x) {
    if (x != x) return x;
    if (x < 2.5) return 1.0 - orc_erf(x);
    if (x > 27.3) return 0.0;
    return erfc_tail(x);
}

/* gelu (nn.hpp:474-478): 0.5 x erfc(-x / sqrt 2) in double, rounded once. */
float orc_gelu(float x) {
    const double inv_sqrt2 = 7.07106781186547524401e-01;
    const double d = x;
    return (float)(0.5 * d * orc_erfc(-d * inv_sqrt2));
}

/* gelu_backward (grad.hpp:165-172): dy (0.5 erfc(-x / sqrt 2) + x e^(-x^2 / 2) / sqrt(2 pi)), rounded once. */
float orc_gelu_backward(float x, float dy) {
    const double inv_sqrt2 = 7.07106781186547524401e-01;
    const double inv_sqrt_2pi = 3.98942280401432677940e-01;
    const double d = x;
    const double slope = 0.5 * orc_erfc(-d * inv_sqrt2) + d * orc_exp(-0.5 * d * d) * inv_sqrt_2pi;
    return (float)((double)dy * slope);
}

/* layer_norm (nn.hpp:412-432): mean and the centred sum of squares over the row ascending, inv_std = 1 / sqrt(. /
 * dim + eps); out = f32((x - mean) inv_std w + b). */
void orc_layer_norm(const float* x, const float* w, const float* b, float* out, size_t rows, size_t dim, double eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        double total = 0.0;
        for (size_t i = 0; i < dim; ++i) total += (double)xr[i];
        const double mean = total / (double)dim;
        double sum_sq = 0.0;
        for (size_t i = 0; i < dim; ++i) {
            const double c = (double)xr[i] - mean;
            sum_sq += c * c;
        }
        const double inv_std = 1.0 / sqrt(sum_sq / (double)dim + eps);
        for (size_t i = 0; i < dim; ++i) {
            const double scaled = ((double)xr[i] - mean) * inv_std * (double)w[i];
            out[r * dim + i] = (float)(scaled + (double)b[i]);
        }
    }
}

/* layer_norm_backward (grad.hpp:112-163): per row the forward's mean and inv_std, xhat = (x - mean) inv_std,
 * g = w dy; sums of g and g xhat over the row ascending; dx = f32(inv_std (g - sum g / dim - xhat sum(g xhat) / dim));
 * dw = f32(sum over rows ascending of dy xhat), db = f32(sum of dy). */
void orc_layer_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                             size_t rows, size_t dim, double eps) {
    double* dw_acc = (double*)calloc(dim ? dim : 1, sizeof(double));
    double* db_acc = (double*)calloc(dim ? dim : 1, sizeof(double));
    double* xhat = (double*)malloc((dim ? dim : 1) * sizeof(double));
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        const float* dyr = dy + r * dim;
        double total = 0.0;
        for (size_t i = 0; i < dim; ++i) total += (double)xr[i];
        const double mean = total / (double)dim;
        double sum_sq = 0.0;
        for (size_t i = 0; i < dim; ++i) {
            const double c = (double)xr[i] - mean;
            sum_sq += c * c;
        }
        const double inv_std = 1.0 / sqrt(sum_sq / (double)dim + eps);
        double g_sum = 0.0, gx_sum = 0.0;
        for (size_t i = 0; i < dim; ++i) {
            xhat[i] = ((double)xr[i] - mean) * inv_std;
            const double g = (double)w[i] * (double)dyr[i];
            g_sum += g;
            gx_sum += g * xhat[i];
            dw_acc[i] += (double)dyr[i] * xhat[i];
            db_acc[i] += (double)dyr[i];
        }
        if (dx) {
            const double g_mean = g_sum / (double)dim;
            const double gx_mean = gx_sum / (double)dim;
            for (size_t i = 0; i < dim; ++i) {
                const double g = (double)w[i] * (double)dyr[i];
                dx[r * dim + i] = (float)(inv_std * (g - g_mean - xhat[i] * gx_mean));
            }
        }
    }
    for (size_t i = 0; i < dim; ++i) {
        if (dw) dw[i] = (float)dw_acc[i];
        if (db) db[i] = (float)db_acc[i];
    }
    free(dw_acc);
    free(db_acc);
    free(xhat);
}

/* biased_attention (nn.hpp:827-856): scores (q k + bias) scale, then attention_finish without soft-cap. q [q_len,
 * heads, head_dim], k [kv_len, heads, head_dim], v [kv_len, heads, value_dim], bias [heads, q_len, kv_len]. */
void orc_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out, size_t q_len,
                          size_t kv_len, size_t heads, size_t head_dim, size_t value_dim, double scale) {
    double* s = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* acc = (double*)malloc((value_dim ? value_dim : 1) * sizeof(double));
    for (size_t t = 0; t < q_len; ++t)
        for (size_t h = 0; h < heads; ++h) {
            float* oh = out + (t * heads + h) * value_dim;
            if (kv_len == 0) {
                for (size_t i = 0; i < value_dim; ++i) oh[i] = 0.0f;
                continue;
            }
            const float* qh = q + (t * heads + h) * head_dim;
            const float* bh = bias + (h * q_len + t) * kv_len;
            for (size_t j = 0; j < kv_len; ++j) {
                const float* kj = k + (j * heads + h) * head_dim;
                double d = 0.0;
                for (size_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
                s[j] = (d + (double)bh[j]) * scale;
            }
            double max = s[0];
            for (size_t j = 1; j < kv_len; ++j)
                if (s[j] > max) max = s[j];
            double total = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                s[j] = orc_exp(s[j] - max);
                total += s[j];
            }
            for (size_t i = 0; i < value_dim; ++i) acc[i] = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                const float* vj = v + (j * heads + h) * value_dim;
                for (size_t i = 0; i < value_dim; ++i) acc[i] += s[j] * (double)vj[i];
            }
            const double inv = 1.0 / total;
            for (size_t i = 0; i < value_dim; ++i) oh[i] = (float)(acc[i] * inv);
        }
    free(s);
    free(acc);
}

/* biased_attention_weights (interp.hpp:79-121): biased_attention's probabilities, f32(exp(s_j - max) (1 / total))
 * per (t, h) into out [q_len, heads, kv_len]; nothing is written when kv_len is 0. */
void orc_biased_attention_weights(const float* q, const float* k, const float* bias, float* out, size_t q_len,
                                  size_t kv_len, size_t heads, size_t head_dim, double scale) {
    if (kv_len == 0) return;
    double* s = (double*)malloc(kv_len * sizeof(double));
    for (size_t t = 0; t < q_len; ++t)
        for (size_t h = 0; h < heads; ++h) {
            const float* qh = q + (t * heads + h) * head_dim;
            const float* bh = bias + (h * q_len + t) * kv_len;
            float* row = out + (t * heads + h) * kv_len;
            for (size_t j = 0; j < kv_len; ++j) {
                const float* kj = k + (j * heads + h) * head_dim;
                double d = 0.0;
                for (size_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
                s[j] = (d + (double)bh[j]) * scale;
            }
            double max = s[0];
            for (size_t j = 1; j < kv_len; ++j)
                if (s[j] > max) max = s[j];
            double total = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                s[j] = orc_exp(s[j] - max);
                total += s[j];
            }
            const double inv = 1.0 / total;
            for (size_t j = 0; j < kv_len; ++j) row[j] = (float)(s[j] * inv);
        }
    free(s);
}

/* biased_attention_backward (grad.hpp:300-389): per (t, h), t then h ascending: p recomputed (scores, max, exp,
 * total, times 1 / total), dp_j = dout . v_j, D = sum p dp, ds = p (dp - D) scale (dbias = f32(ds)), dq = sum_j ds
 * k_j; dk[j] += ds q, dv[j] += p dout in double, rounded once at the end. */
void orc_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                   const float* dout, float* dq, float* dk, float* dv, float* dbias, size_t q_len,
                                   size_t kv_len, size_t heads, size_t head_dim, size_t value_dim, double scale) {
    double* probs = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* dprobs = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    double* dq_acc = (double*)malloc((head_dim ? head_dim : 1) * sizeof(double));
    double* dk_acc = (double*)calloc(kv_len * heads * head_dim + 1, sizeof(double));
    double* dv_acc = (double*)calloc(kv_len * heads * value_dim + 1, sizeof(double));
    for (size_t t = 0; t < q_len; ++t)
        for (size_t h = 0; h < heads; ++h) {
            const float* qh = q + (t * heads + h) * head_dim;
            const float* bh = bias + (h * q_len + t) * kv_len;
            const float* doh = dout + (t * heads + h) * value_dim;
            float* dqh = dq + (t * heads + h) * head_dim;
            float* dbh = dbias + (h * q_len + t) * kv_len;
            if (kv_len == 0) {
                for (size_t i = 0; i < head_dim; ++i) dqh[i] = 0.0f;
                continue;
            }
            double max = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                const float* kj = k + (j * heads + h) * head_dim;
                double d = 0.0;
                for (size_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
                probs[j] = (d + (double)bh[j]) * scale;
                if (j == 0 || probs[j] > max) max = probs[j];
            }
            double total = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                probs[j] = orc_exp(probs[j] - max);
                total += probs[j];
            }
            const double inv = 1.0 / total;
            double weighted = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                probs[j] *= inv;
                const float* vj = v + (j * heads + h) * value_dim;
                double d = 0.0;
                for (size_t i = 0; i < value_dim; ++i) d += (double)doh[i] * (double)vj[i];
                dprobs[j] = d;
                weighted += probs[j] * d;
            }
            for (size_t i = 0; i < head_dim; ++i) dq_acc[i] = 0.0;
            for (size_t j = 0; j < kv_len; ++j) {
                const double ds = probs[j] * (dprobs[j] - weighted) * scale;
                dbh[j] = (float)ds;
                const float* kj = k + (j * heads + h) * head_dim;
                double* dkj = dk_acc + (j * heads + h) * head_dim;
                double* dvj = dv_acc + (j * heads + h) * value_dim;
                for (size_t i = 0; i < head_dim; ++i) {
                    dq_acc[i] += ds * (double)kj[i];
                    dkj[i] += ds * (double)qh[i];
                }
                for (size_t i = 0; i < value_dim; ++i) dvj[i] += probs[j] * (double)doh[i];
            }
            for (size_t i = 0; i < head_dim; ++i) dqh[i] = (float)dq_acc[i];
        }
    for (size_t i = 0; i < kv_len * heads * head_dim; ++i) dk[i] = (float)dk_acc[i];
    for (size_t i = 0; i < kv_len * heads * value_dim; ++i) dv[i] = (float)dv_acc[i];
    free(probs);
    free(dprobs);
    free(dq_acc);
    free(dk_acc);
    free(dv_acc);
}

/* rope_inv_freq with default scaling (numerics.py:267-297): theta^(-2i/dim) = exp(-(2i/dim) log theta). */
void orc_rope_inv_freq(size_t rotary_dim, double theta, double* out) {
    const double log_theta = orc_log(theta);
    for (size_t i = 0; i < rotary_dim / 2; ++i) {
        const double frac = (double)(2 * (int64_t)i) / (double)rotary_dim;
        out[i] = orc_exp(-frac * log_theta);
    }
}

/* rope_inv_freq with rope_scaling (numerics.py:267-349 and _yarn 325-349), every step in the Python code's double
 * operation order: Python ints divide as correctly rounded doubles, min/max/floor/ceil as written. */
int orc_rope_inv_freq_scaled(size_t rotary_dim, double theta, const orc_rope_scaling* sc, double* out) {
    const size_t pairs = rotary_dim / 2;
    const double log_theta = orc_log(theta);
    for (size_t i = 0; i < pairs; ++i) out[i] = orc_exp(-((double)(2 * (int64_t)i) / (double)rotary_dim) * log_theta);
    const int64_t kind = sc ? sc->kind : 0;
    const double pi = 3.141592653589793; /* math.pi */
    if (kind == 0) return 0;
    if (kind == 1) {
        for (size_t i = 0; i < pairs; ++i) out[i] = out[i] / sc->factor;
        return 0;
    }
    if (kind == 2) {
        const double low = sc->low_freq_factor, high = sc->high_freq_factor, original = sc->original;
        const double low_freq_wavelen = original / low, high_freq_wavelen = original / high;
        for (size_t i = 0; i < pairs; ++i) {
            const double f = out[i];
            const double wavelen = 2 * pi / f;
            if (wavelen < high_freq_wavelen) {
                out[i] = f;
            } else if (wavelen > low_freq_wavelen) {
                out[i] = f / sc->factor;
            } else {
                const double smooth = (original / wavelen - low) / (high - low);
                out[i] = (1 - smooth) * f / sc->factor + smooth * f;
            }
        }
        return 0;
    }
    if (kind == 3) {
        for (size_t i = 0; i < pairs; ++i) out[i] = out[i] / sc->factors[i];
        return 0;
    }
    if (kind == 4) {
        const double dim = (double)rotary_dim, original = sc->original;
        double low = dim * orc_log(original / (sc->beta_fast * 2 * pi)) / (2 * log_theta);
        double high = dim * orc_log(original / (sc->beta_slow * 2 * pi)) / (2 * log_theta);
        if (sc->truncate) {
            low = floor(low);
            high = ceil(high);
        }
        if (low < 0) low = 0; /* max(low, 0) */
        if (high > dim - 1) high = dim - 1; /* min(high, dim - 1) */
        if (low == high) high += 0.001;
        for (size_t i = 0; i < pairs; ++i) {
            double ramp = ((double)(int64_t)i - low) / (high - low);
            if (ramp < 0.0) ramp = 0.0;
            if (ramp > 1.0) ramp = 1.0;
            const double f = out[i];
            out[i] = f / sc->factor * ramp + f * (1 - ramp);
        }
        return 0;
    }
    return 1;
}

/* ---- the oracle's kernel table ---- */
static void silu_n(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_silu(x[i]);
}
static void silu_backward_n(const float* x, const float* dy, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_silu_backward(x[i], dy[i]);
}

static void gelu_tanh_n(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_gelu_tanh(x[i]);
}
static void gelu_tanh_backward_n(const float* x, const float* dy, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_gelu_tanh_backward(x[i], dy[i]);
}
/* softcap (nn.hpp:457-461): cap tanh(x / cap) in double, rounded once. */
static void softcap_n(const float* x, float* out, size_t n, double cap) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)(cap * orc_tanh((double)x[i] / cap));
}
static void softcap_backward_n(const float* x, const float* dy, float* out, size_t n, double cap) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_softcap_backward(x[i], dy[i], cap);
}

static const orc_ops default_ops = {
    orc_linear, orc_linear_backward, orc_rms_norm, orc_rms_norm_backward, orc_rope, orc_attention,
    orc_attention_backward, silu_n, orc_swiglu, silu_backward_n, orc_cross_entropy, orc_embedding_backward,
    orc_sum_squares, orc_adamw_step, orc_softmax, orc_moe_route, orc_moe_route_backward, orc_column_mean, orc_dot,
    gelu_tanh_n, gelu_tanh_backward_n, softcap_n, softcap_backward_n,
};

const orc_ops* orc_default_ops(void) { return &default_ops; }
