// ft_libm.hpp -- f32 tanh and exp that return the bits of glibc 2.35's
// tanhf / expf on x86_64, the functions Rust's f32::tanh and f32::exp call on
// Linux. ft-core computes GELU with f32::tanh (ft-model/src/lib.rs:436) and the
// routing weights with f32::exp (ft-model/src/lib.rs:1495), so the kernels use
// these to produce the same activation q8 blocks and routing weights.
//
// The same source compiles for the host (the CPU test sweeps it against the
// system libm over every f32 input of each domain) and for gfx950. Every step
// is an IEEE basic operation (add, sub, mul, div, fma, int<->float
// conversion), written out in the order of the published algorithm, so both
// targets round identically. Callers compile with -ffp-contract=off.
//
//   tanhf: the fdlibm algorithm (Sun Microsystems, 1993; single-precision
//          version by Cygnus Support) that glibc ships as its generic
//          flt-32 tanhf: for |x| < 22, tanh(|x|) = -t/(t+2) with
//          t = expm1(-2|x|) below 1 and 1 - 2/(expm1(2|x|)+2) from 1 on.
//   expm1f: fdlibm's single-precision expm1 (as tanhf uses it): x = k*ln2
//          + r (ln2 in two parts), then expm1(r) from a rational
//          approximation R1(r^2) of (r/2)*coth(r/2) by a degree-5 polynomial
//          in r^2/2, then the result rebuilt from k.
//   expf:  glibc's double-precision-evaluated expf (Szabolcs Nagy, ARM,
//          2017; glibc 2.27+): z = x*32/ln2, k = round(z), r = z - k,
//          exp(x) = 2^(k/32) * p(r) with 2^(i/32) from a 32-entry table and
//          p a degree-3 polynomial. On x86_64 glibc runs its FMA build on
//          FMA-capable hosts, so the polynomial's three multiply-adds are
//          fused here too.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FT_LIBM_FN __host__ __device__ __forceinline__
#define FT_LIBM_MEMBER __host__ __device__ __forceinline__
#else
#define FT_LIBM_FN static inline
#define FT_LIBM_MEMBER inline
#endif

namespace ft {
namespace libm {

FT_LIBM_FN uint32_t bits_f(float x) {
    uint32_t u;
    __builtin_memcpy(&u, &x, 4);
    return u;
}
FT_LIBM_FN float from_bits_f(uint32_t u) {
    float x;
    __builtin_memcpy(&x, &u, 4);
    return x;
}
FT_LIBM_FN uint64_t bits_d(double x) {
    uint64_t u;
    __builtin_memcpy(&u, &x, 8);
    return u;
}
FT_LIBM_FN double from_bits_d(uint64_t u) {
    double x;
    __builtin_memcpy(&x, &u, 8);
    return x;
}

// fdlibm single-precision constants (hex: IEEE bits).
struct Expm1Const {
    static constexpr float ln2_hi = 6.9313812256e-01f;   // 0x3f317180: low bits clear, so t*ln2_hi is exact
    static constexpr float ln2_lo = 9.0580006145e-06f;   // 0x3717f7d1
    static constexpr float invln2 = 1.4426950216e+00f;   // 0x3fb8aa3b
    // R1(r^2) = 1 + Q1*h + ... + Q5*h^5 with h = r^2/2 (f32 roundings of
    // fdlibm's double coefficients)
    static constexpr float Q1 = -3.3333335072e-02f;      // 0xbd088889
    static constexpr float Q2 = 1.5873016091e-03f;       // 0x3ad00d01
    static constexpr float Q3 = -7.9365076090e-05f;      // 0xb8a670cd
    static constexpr float Q4 = 4.0082177293e-06f;       // 0x36867e54
    static constexpr float Q5 = -2.0109921195e-07f;      // 0xb457edbb
};

// fdlibm's expm1f on the arguments tanhf gives it: a in [2, 44) or
// [-2, -2^-54], so none of its special cases (NaN, inf, overflow, the -1
// saturation below -27*ln2) arise. Straight-line: the reduction's three
// forms and the result's reconstructions for every k are computed and the
// one fdlibm's branches would take is selected, so a wavefront runs one
// path instead of every branch taken by some lane. The arithmetic of the
// selected form is fdlibm's, operation for operation.
FT_LIBM_FN float expm1f_tanh_args(float x) {
    using C = Expm1Const;
    const uint32_t bx = bits_f(x);
    const bool neg = (bx >> 31) != 0;
    const uint32_t ax = bx & 0x7fffffffu;
    // reduction x = k*ln2 + (hi - lo), applied when |x| > ln2/2
    const bool reduce = ax > 0x3eb17218u;
    const bool k1 = ax < 0x3f851592u;        // |x| < 3ln2/2: k = +-1 with the plain ln2 parts
    const int kn = (int)(C::invln2 * x + (neg ? -0.5f : 0.5f));  // truncating conversion
    const float tn = (float)kn;
    const float hi_n = x - tn * C::ln2_hi, lo_n = tn * C::ln2_lo;
    const float hi_1 = neg ? x + C::ln2_hi : x - C::ln2_hi;
    const float lo_1 = neg ? -C::ln2_lo : C::ln2_lo;
    const float hi = k1 ? hi_1 : hi_n, lo = k1 ? lo_1 : lo_n;
    const int k = reduce ? (k1 ? (neg ? -1 : 1) : kn) : 0;
    const float xr = hi - lo;
    const float c = reduce ? (hi - xr) - lo : 0.0f;
    const float r = reduce ? xr : x;
    // expm1(r) = r + r^2/2 + r^3/2 * (3 - (R1 + R1*r/2)) / (6 - r*(3 - R1*r/2))
    const float hfx = 0.5f * r;
    const float hxs = r * hfx;
    const float r1 = 1.0f + hxs * (C::Q1 + hxs * (C::Q2 + hxs * (C::Q3 + hxs * (C::Q4 + hxs * C::Q5))));
    const float t = 3.0f - r1 * hfx;
    const float e = hxs * ((r1 - t) / (6.0f - r * t));
    // reconstructions, by k
    const float res_k0 = r - (r * e - hxs);                       // k == 0
    const float e2 = (r * (e - c) - c) - hxs;
    const float res_m1 = 0.5f * (r - e2) - 0.5f;                  // k == -1
    const float res_p1 = r < -0.25f ? -2.0f * (e2 - (r + 0.5f))   // k == 1
                                    : 1.0f + 2.0f * (r - e2);
    const uint32_t ksh = (uint32_t)k << 23;                       // adds k to an exponent field
    const float y_far = from_bits_f(bits_f(1.0f - (e2 - r)) + ksh);
    const float res_far = y_far - 1.0f;                           // k <= -2 or k > 56
    const int kl = k < 1 ? 1 : (k > 22 ? 22 : k);                 // shift amounts kept in range
    const float one_m = from_bits_f(0x3f800000u - (0x1000000u >> kl));  // 1 - 2^-k
    const float res_lo = from_bits_f(bits_f(one_m - (e2 - r)) + ksh);  // 2 <= k < 23
    const int kh = k < 23 ? 23 : (k > 56 ? 56 : k);
    const float two_mk = from_bits_f((uint32_t)(0x7f - kh) << 23);      // 2^-k
    const float res_hi = from_bits_f(bits_f((r - (e2 + two_mk)) + 1.0f) + ksh);  // 23 <= k <= 56
    float res = res_far;
    if (k >= 2 && k < 23) res = res_lo;
    if (k >= 23 && k <= 56) res = res_hi;
    if (k == 1) res = res_p1;
    if (k == -1) res = res_m1;
    if (k == 0) res = res_k0;
    if (ax < 0x33000000u) res = x;                                // |x| < 2^-25: x itself
    return res;
}

// tanhf(x), every f32 input: fdlibm's formulas, with the two expm1f calls
// (of 2|x| from |x| >= 1, of -2|x| below) as one call on the selected
// argument and the two quotients as one division.
FT_LIBM_FN float tanhf_glibc(float x) {
    const uint32_t bx = bits_f(x);
    const uint32_t ax = bx & 0x7fffffffu;
    const bool neg = (bx >> 31) != 0;
    const bool mid = ax < 0x41b00000u;       // |x| < 22 (false for inf and NaN)
    const float a = mid ? from_bits_f(ax) : 1.0f;  // lanes overridden below get an in-range argument
    const bool ge1 = ax >= 0x3f800000u;      // |x| >= 1
    const float tm = expm1f_tanh_args(ge1 ? 2.0f * a : -2.0f * a);
    const float q = (ge1 ? 2.0f : -tm) / (tm + 2.0f);
    float z = ge1 ? 1.0f - q : q;
    if (!mid) z = 1.0f;                      // |x| >= 22: 1 - tiny rounds to 1
    if (ax < 0x24000000u) z = a * (1.0f + a);  // |x| < 2^-55 (and +-0): x*(1+x) = x
    z = neg ? -z : z;
    if (ax >= 0x7f800000u) z = neg ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;  // +-inf -> +-1, NaN -> NaN
    return z;
}

// 2^(i/32) as IEEE double bits minus i << 47, so that adding k << 47 for
// k = 32m + i gives 2^(k/32) (the exponent field absorbs m). Entries are the
// correctly rounded doubles of 2^(i/32).
struct Exp2Table {
    uint64_t t[32];
};
FT_LIBM_FN constexpr Exp2Table exp2_table() {
    return Exp2Table{{
        0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
        0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
        0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
        0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
        0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
        0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
        0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
        0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
    }};
}

// expf(x), every f32 input. The table read goes through `tab`, anything
// indexable by 0..31 that holds exp2_table() (a persistent kernel passes a
// copy in LDS).
template <typename Tab>
FT_LIBM_FN float expf_glibc_t(float x, const Tab& tab) {
    constexpr double N = 32.0;
    constexpr double inv_ln2_n = 0x1.71547652b82fep+0 * N;
    constexpr double shift = 0x1.8p+52;       // z + shift rounds z to an integer in the low mantissa bits
    constexpr double c0 = 0x1.c6af84b912394p-5 / N / N / N;
    constexpr double c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    constexpr double c2 = 0x1.62e42ff0c52d6p-1 / N;
    const uint32_t top = (bits_f(x) >> 20) & 0x7ff;  // top 12 bits without the sign
    if (top >= 0x42b) {                      // |x| >= 88 or NaN/inf
        if (bits_f(x) == 0xff800000u) return 0.0f;
        if (top >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    // z = x*32/ln2 feeds two additions, and both are fused with the product
    // (GCC contracts every use of a product that only feeds adds): kd =
    // round(z) through the shift, r = z - kd from the unrounded product.
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);  // round to nearest, ties to even
    const uint64_t ki = bits_d(kd);
    kd = kd - shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = from_bits_d(t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

struct Exp2TableRef {
    FT_LIBM_MEMBER uint64_t operator[](uint64_t i) const { return exp2_table().t[i]; }
};

FT_LIBM_FN float expf_glibc(float x) { return expf_glibc_t(x, Exp2TableRef{}); }

}  // namespace libm
}  // namespace ft
