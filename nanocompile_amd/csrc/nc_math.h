// expf, sinf and cosf that compute the same bits on the GPU and on the host.
//
// The reference calls the C library's expf, sinf and cosf (codegen_c.py:58),
// and the GPU's own math library rounds differently in rare cases. Here each
// function is written once, in plain C with only IEEE double operations
// (add, subtract, multiply; no division, no fused multiply-add: both gcc and
// hipcc build it with -ffp-contract=off), so gcc on the host and hipcc on
// gfx950 produce identical results, and the host oracle can replay a GPU
// kernel bit for bit.
//
// Method (Cody and Waite's argument reduction, then a Taylor polynomial):
//   exp(x) = 2^k * exp(r),   k = nearest(x / ln 2),     |r| <= ln(2) / 2
//   sin/cos(x): k = nearest(x * 2 / pi), r = x - k * pi / 2 (two-part pi / 2),
//   then sin(r) or cos(r) by quadrant, |r| <= pi / 4.
// Everything runs in double, so the result before the final rounding to
// float carries a relative error near 1e-15, and the float result is the
// correctly rounded one except when the exact value lies within ~1e-15 of a
// rounding boundary. Tests hold all three within one ulp of glibc's, and
// equal to it on nearly every input.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define NC_MATH_FN __host__ __device__ __forceinline__
#else
#define NC_MATH_FN static inline
#endif

NC_MATH_FN double nc_pow2i(int k) {
    // 2^k as a double, for -1022 <= k <= 1023: the exponent field directly.
    union { uint64_t u; double d; } v;
    v.u = (uint64_t)(k + 1023) << 52;
    return v.d;
}

NC_MATH_FN double nc_nearest(double x) {
    // Round to nearest integer, ties away from zero (which tie does not matter
    // here: either neighbour keeps |r| within the polynomial's range). trunc
    // is the conversion to int64 and back for every |x| < 2^63, in one
    // instruction on the GPU rather than an emulated 64-bit conversion.
    return __builtin_trunc(x + (x >= 0.0 ? 0.5 : -0.5));
}

NC_MATH_FN float nc_expf(float xf) {
    // The special cases are chosen at the end, so the GPU runs one straight
    // path with no divergent branch; their operand is replaced by 0 first.
    const int nan = xf != xf;
    const int big = xf > 100.0f;                   // past FLT_MAX: +inf (up to 100 the
                                                   // double result rounds to inf itself)
    const int tiny = xf < -104.0f;                 // below half the least subnormal: 0
    const double x = (nan | big | tiny) ? 0.0 : (double)xf;
    const double inv_ln2 = 1.4426950408889634;
    const double ln2_hi = 6.93147180369123816490e-01;   // 33 significant bits: k * ln2_hi is exact
    const double ln2_lo = 1.90821492927058770002e-10;
    const double k = nc_nearest(x * inv_ln2);
    const double r = (x - k * ln2_hi) - k * ln2_lo;
    // exp(r), |r| <= 0.3466: Taylor to r^13 (truncation < 3e-17 relative),
    // Horner's steps as a multiply and an add each (measured on MI355X: the
    // fused double multiply-add form made the prefill attention kernel, where
    // 7 of these chains run side by side, 6% slower)
    double p = 1.0 / 6227020800.0;                 // 1/13!
    p = p * r + 1.0 / 479001600.0;                 // 1/12!
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
    const int ki = (int)k;
    // 2^k may be subnormal in float but never in double (k >= -150)
    const float y = (float)(p * nc_pow2i(ki));
    return nan ? xf : big ? (float)(1e300 * 1e300) : tiny ? 0.0f : y;
}

// sin(r) and cos(r) for |r| <= pi/4 + a little, Taylor to r^17 / r^18
// (truncation below 1e-19). Horner in r^2 from the highest term.
NC_MATH_FN double nc_sin_poly(double r) {
    const double r2 = r * r;
    double p = 1.0 / 355687428096000.0;            // +1/17!
    p = p * r2 - 1.0 / 1307674368000.0;            // -1/15!
    p = p * r2 + 1.0 / 6227020800.0;               // +1/13!
    p = p * r2 - 1.0 / 39916800.0;                 // -1/11!
    p = p * r2 + 1.0 / 362880.0;                   // +1/9!
    p = p * r2 - 1.0 / 5040.0;                     // -1/7!
    p = p * r2 + 1.0 / 120.0;                      // +1/5!
    p = p * r2 - 1.0 / 6.0;                        // -1/3!
    return r + r * (r2 * p);
}

NC_MATH_FN double nc_cos_poly(double r) {
    const double r2 = r * r;
    double p = -1.0 / 6402373705728000.0;          // -1/18!
    p = p * r2 + 1.0 / 20922789888000.0;           // +1/16!
    p = p * r2 - 1.0 / 87178291200.0;              // -1/14!
    p = p * r2 + 1.0 / 479001600.0;                // +1/12!
    p = p * r2 - 1.0 / 3628800.0;                  // -1/10!
    p = p * r2 + 1.0 / 40320.0;                    // +1/8!
    p = p * r2 - 1.0 / 720.0;                      // -1/6!
    p = p * r2 + 1.0 / 24.0;                       // +1/4!
    p = p * r2 - 0.5;                              // -1/2!
    return 1.0 + r2 * p;
}

// Reduces x to r in [-pi/4, pi/4] with x = q * pi/2 + r; returns q mod 4.
// Valid for |x| < 2^20 * pi/2 (angles to ~1.6e6 radians): q * pio2_1 is exact.
NC_MATH_FN int nc_reduce_pio2(double x, double *r) {
    const double two_over_pi = 6.36619772367581382433e-01;
    const double pio2_1 = 1.57079632673412561417e+00;   // first 33 bits of pi/2
    const double pio2_1t = 6.07710050650619224932e-11;  // pi/2 - pio2_1
    const double q = nc_nearest(x * two_over_pi);
    *r = (x - q * pio2_1) - q * pio2_1t;
    return ((int)(int64_t)q) & 3;
}

NC_MATH_FN float nc_sinf(float xf) {
    if (xf != xf) return xf;
    if (xf - xf != 0.0f) return xf - xf;           // +-inf: NaN
    if (xf == 0.0f) return xf;                     // keeps the sign of zero
    double r;
    const int q = nc_reduce_pio2((double)xf, &r);
    double v;
    switch (q) {
        case 0: v = nc_sin_poly(r); break;
        case 1: v = nc_cos_poly(r); break;
        case 2: v = -nc_sin_poly(r); break;
        default: v = -nc_cos_poly(r); break;
    }
    return (float)v;
}

NC_MATH_FN float nc_cosf(float xf) {
    if (xf != xf) return xf;
    if (xf - xf != 0.0f) return xf - xf;           // +-inf: NaN
    double r;
    const int q = nc_reduce_pio2((double)xf, &r);
    double v;
    switch (q) {
        case 0: v = nc_cos_poly(r); break;
        case 1: v = -nc_sin_poly(r); break;
        case 2: v = -nc_cos_poly(r); break;
        default: v = nc_sin_poly(r); break;
    }
    return (float)v;
}
