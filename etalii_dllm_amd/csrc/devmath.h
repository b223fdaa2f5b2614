// Device restatement of the reference's portable transcendentals (cpp/include/dllm/math.hpp), so every exp, log, sin,
// cos, tanh and sigmoid on the GPU returns the same bits as the reference CPU kernels. Built from + - * / only, in
// the same operation order; the library is compiled with -ffp-contract=off so no multiply-add is fused. The Taylor
// and odd-series coefficients and the two-part ln2 / three-part pi/2 constants are the ones those series and
// reductions require; they must match the reference exactly for the results to match.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dllm_hip {

__host__ __device__ inline double bits_double(uint64_t b) { return __builtin_bit_cast(double, b); }
__host__ __device__ inline uint64_t double_bits(double x) { return __builtin_bit_cast(uint64_t, x); }

__host__ __device__ inline double pow2_bits(int k) { return bits_double(static_cast<uint64_t>(k + 1023) << 52); }

// e^x (math.hpp:64-109).
__host__ __device__ inline double dexp(double x) {
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double inv_ln2 = 1.44269504088896338700e+00;
    if (x != x) return x;
    if (x > 709.78) return bits_double(0x7ff0000000000000ULL);
    if (x < -745.2) return 0.0;
    const double kd = x * inv_ln2;
    const int k = static_cast<int>(kd >= 0 ? kd + 0.5 : kd - 0.5);
    const double r = (x - k * ln2_hi) - k * ln2_lo;
    double p = 1.0 / 6227020800.0;  // 1/13!
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    int e = k;
    while (e > 1023) {
        p *= pow2_bits(1023);
        e -= 1023;
    }
    while (e < -1022) {
        p *= pow2_bits(-1022);
        e += 1022;
    }
    return p * pow2_bits(e);
}

// log x (math.hpp:113-162).
__host__ __device__ inline double dlog(double x) {
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double sqrt_half = 7.07106781186547524401e-01;
    if (x != x || x < 0.0) return bits_double(0x7ff8000000000000ULL);
    if (x == 0.0) return bits_double(0xfff0000000000000ULL);
    if (x == bits_double(0x7ff0000000000000ULL)) return x;
    int e = 0;
    if (x < 2.2250738585072014e-308) {
        x *= pow2_bits(54);
        e -= 54;
    }
    uint64_t bits = double_bits(x);
    e += static_cast<int>((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL;
    double m = bits_double(bits);
    if (m >= 2.0 * sqrt_half) {
        m *= 0.5;
        e += 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 25.0;
    p = p * s2 + 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    const double log_m = 2.0 * s + 2.0 * s * s2 * p;
    return (e * ln2_hi + log_m) + e * ln2_lo;
}

__device__ inline double dsin_kernel(double r) {
    const double r2 = r * r;
    double p = -1.0 / 1307674368000.0;  // -1/15!
    p = p * r2 + 1.0 / 6227020800.0;
    p = p * r2 - 1.0 / 39916800.0;
    p = p * r2 + 1.0 / 362880.0;
    p = p * r2 - 1.0 / 5040.0;
    p = p * r2 + 1.0 / 120.0;
    p = p * r2 - 1.0 / 6.0;
    return r + r * r2 * p;
}

__device__ inline double dcos_kernel(double r) {
    const double r2 = r * r;
    double p = 1.0 / 20922789888000.0;  // 1/16!
    p = p * r2 - 1.0 / 87178291200.0;
    p = p * r2 + 1.0 / 479001600.0;
    p = p * r2 - 1.0 / 3628800.0;
    p = p * r2 + 1.0 / 40320.0;
    p = p * r2 - 1.0 / 720.0;
    p = p * r2 + 1.0 / 24.0;
    return (1.0 - 0.5 * r2) + r2 * r2 * p;
}

// x = n pi/2 + r (math.hpp:194-216).
__device__ inline double dreduce_half_pi(double x, int* quadrant) {
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
        n = nd >= 0 ? static_cast<double>(static_cast<long long>(nd + 0.5))
                    : static_cast<double>(static_cast<long long>(nd - 0.5));
    }
    const double r = (((x - n * pio2_1) - n * pio2_2) - n * pio2_3) - n * pio2_3t;
    *quadrant = (n < two_62 && n > -two_62) ? static_cast<int>(static_cast<long long>(n) & 3) : 0;
    return r;
}

__device__ inline bool dnonfinite(double x) {
    return x != x || x == __longlong_as_double(0x7ff0000000000000LL) ||
           x == __longlong_as_double(static_cast<long long>(0xfff0000000000000ULL));
}

__device__ inline double dsin(double x) {
    if (dnonfinite(x)) return __longlong_as_double(0x7ff8000000000000LL);
    int q;
    const double r = dreduce_half_pi(x, &q);
    switch (q) {
        case 0: return dsin_kernel(r);
        case 1: return dcos_kernel(r);
        case 2: return -dsin_kernel(r);
        default: return -dcos_kernel(r);
    }
}

__device__ inline double dcos(double x) {
    if (dnonfinite(x)) return __longlong_as_double(0x7ff8000000000000LL);
    int q;
    const double r = dreduce_half_pi(x, &q);
    switch (q) {
        case 0: return dcos_kernel(r);
        case 1: return -dsin_kernel(r);
        case 2: return -dcos_kernel(r);
        default: return dsin_kernel(r);
    }
}

// The sine and cosine of pos x freq, the same values as dsin and dcos of that product: one reduction, both
// polynomials, and the quadrant picks which one (and its sign) each result takes, with no divergent branch.
__device__ inline void dsincos(double pos, double freq, double* sin_out, double* cos_out) {
    const double x = pos * freq;
    if (dnonfinite(x)) {
        *sin_out = *cos_out = __longlong_as_double(0x7ff8000000000000LL);
        return;
    }
    int q;
    const double r = dreduce_half_pi(x, &q);
    const double ps = dsin_kernel(r), pc = dcos_kernel(r);
    const double s = (q & 1) ? pc : ps, c = (q & 1) ? ps : pc;
    *sin_out = (q & 2) ? -s : s;
    *cos_out = ((q + 1) & 2) ? -c : c;
}

// tanh (math.hpp:296-319).
__device__ inline double dtanh(double x) {
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
        t = 1.0 - 2.0 / (dexp(2.0 * a) + 1.0);
    }
    return x < 0 ? -t : t;
}

// erfc(a) for a >= 2.5 (math.hpp:332-341): e^(-a^2) / sqrt(pi) / K(a), K the Laplace continued fraction evaluated
// backwards from depth 80.
__host__ __device__ inline double derfc_tail(double a) {
    const double inv_sqrt_pi = 5.64189583547756286948e-01;
    double k = a;
    for (int n = 80; n >= 1; --n) k = a + (0.5 * n) / k;
    return dexp(-a * a) * inv_sqrt_pi / k;
}

// erf (math.hpp:345-370): the 60-term Maclaurin series below 2.5, 1 - erfc_tail(|x|) up to 6, 1 beyond.
__host__ __device__ inline double derf(double x) {
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
        result = 1.0 - derfc_tail(a);
    }
    return x < 0 ? -result : result;
}

// erfc (math.hpp:373-384).
__host__ __device__ inline double derfc(double x) {
    if (x != x) return x;
    if (x < 2.5) return 1.0 - derf(x);
    if (x > 27.3) return 0.0;
    return derfc_tail(x);
}

// sigmoid (math.hpp:322-328).
// Both of the reference's branches as one path (a wave whose lanes differ in sign runs one exp and one division,
// not two of each): x >= 0 gives 1 / (1 + exp(-x)), otherwise exp(x) / (1 + exp(x)); a NaN takes the second form.
__host__ __device__ inline double dsigmoid(double x) {
    const bool nonneg = x >= 0;
    const double e = dexp(nonneg ? -x : x);
    return (nonneg ? 1.0 : e) / (1.0 + e);
}

// silu (nn.hpp:467-470) and its gradient (grad.hpp:177-181), each rounded once to float.
__device__ inline float dsilu(float x) {
    const double d = x;
    return static_cast<float>(d * dsigmoid(d));
}

__device__ inline float dsilu_backward(float x, float dy) {
    const double d = x;
    const double s = dsigmoid(d);
    return static_cast<float>(static_cast<double>(dy) * s * (1.0 + d * (1.0 - s)));
}

}  // namespace dllm_hip
