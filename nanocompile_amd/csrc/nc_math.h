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
//   exp(x) = 2^m * 2^(j / 64) * exp(r),  64 m + j = nearest(64 x / ln 2),
//            |r| <= ln(2) / 128, 2^(j / 64) from a table of 64 doubles
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
#define NC_MATH_TABLE static __device__ __constant__ const
#else
#define NC_MATH_FN static inline
#define NC_MATH_TABLE static const
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

// 2^(j / 64) for j = 0 .. 63, each the double nearest the exact value (written
// as hexadecimal literals so no decimal conversion intervenes).
NC_MATH_TABLE double nc_exp2_64ths[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

NC_MATH_FN float nc_expf(float xf) {
    // The special cases are chosen at the end, so the GPU runs one straight
    // path with no divergent branch; their operand is replaced by 0 first.
    const int nan = xf != xf;
    const int big = xf > 100.0f;                   // past FLT_MAX: +inf (up to 100 the
                                                   // double result rounds to inf itself)
    const int tiny = xf < -104.0f;                 // below half the least subnormal: 0
    const double x = (nan | big | tiny) ? 0.0 : (double)xf;
    const double inv = 0x1.71547652b82fep+6;       // 64 / ln 2
    const double l_hi = 0x1.62e42ffp-7;            // ln 2 / 64 to 29 significant bits: k * l_hi is exact
    const double l_lo = -0x1.718432a1b0e26p-41;    // ln 2 / 64 - l_hi
    const double k = nc_nearest(x * inv);          // |k| <= 9601
    const double r = (x - k * l_hi) - k * l_lo;
    // exp(r), |r| <= ln 2 / 128 = 0.0054: Taylor to r^5 (truncation < 4e-17
    // relative), Horner's steps as a multiply and an add each (measured on
    // MI355X: the fused double multiply-add form made the prefill attention
    // kernel, where 7 of these chains run side by side, 6% slower)
    double p = 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    // k = 64 m + j, 0 <= j < 64: exp(x) = 2^m * 2^(j / 64) * exp(r); 2^m may be
    // subnormal in float but never in double (m >= -151)
    const int ki = (int)k;
    const int j = ki & 63;
    const int m = (ki - j) / 64;
    const float y = (float)(nc_exp2_64ths[j] * p * nc_pow2i(m));
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
