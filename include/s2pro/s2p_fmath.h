/* s2pro MI355X — transcendental functions of the sampling / acceptance rule.
 *
 * The reference sampler (src/slowar/sampling.c:201,216,237-238) calls libm
 * expf/logf, and its own device port is documented as differing from the host
 * at ULP level for sampled draws (src/slowar/slowar_kernels.h:148-149).  To
 * make accept/reject decisions and emitted token ids bit-exact between the
 * host oracle and the HIP kernels, the rule is specified here with its own
 * expf/logf, compiled from this one source by the host C compiler and by hipcc
 * (both with FP contraction off).  Every operation is a basic IEEE-754 binary64
 * operation (+, -, *, /, conversions), so both targets produce identical bits.
 *
 * Method (textbook, no vendor math library):
 *  - exp: Cody-Waite reduction x = k*ln2 + r, |r| <= ln2/2, with ln2 split in
 *    a 32-bit-exact high part and a low part; exp(r) by its Taylor series to
 *    degree 13 (truncation < 5e-18 relative); scaling by 2^k built from the
 *    exponent bits; one final double->float rounding.
 *  - log: x = 2^e * m with m in [sqrt(1/2), sqrt(2)); log m = 2*atanh(s),
 *    s = (m-1)/(m+1), by its odd series to s^25 (|s| <= 0.1716, truncation
 *    < 1e-19); e*ln2 added in two parts; one final double->float rounding.
 * The double-precision intermediate carries ~2^-52 relative error, so the
 * float result equals the correctly rounded expf/logf except when the exact
 * value lies within ~2^-52 (relative) of a float rounding boundary.
 */
#ifndef S2P_FMATH_H
#define S2P_FMATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define S2P_FM_QUAL static __host__ __device__ inline
#else
#define S2P_FM_QUAL static inline
#endif

#if defined(__clang__)
#define S2P_FM_NOCONTRACT _Pragma("clang fp contract(off)")
#else
#define S2P_FM_NOCONTRACT
#endif

S2P_FM_QUAL double s2p_fm_bits2d(uint64_t b) {
    union { uint64_t u; double d; } v;
    v.u = b;
    return v.d;
}
S2P_FM_QUAL uint64_t s2p_fm_d2bits(double d) {
    union { uint64_t u; double d; } v;
    v.d = d;
    return v.u;
}
S2P_FM_QUAL uint32_t s2p_fm_f2bits(float f) {
    union { uint32_t u; float f; } v;
    v.f = f;
    return v.u;
}
S2P_FM_QUAL float s2p_fm_bits2f(uint32_t b) {
    union { uint32_t u; float f; } v;
    v.u = b;
    return v.f;
}

/* exp(x) rounded to float. */
S2P_FM_QUAL float s2p_expf(float xf) {
    S2P_FM_NOCONTRACT
    const uint32_t xb = s2p_fm_f2bits(xf);
    if ((xb & 0x7F800000u) == 0x7F800000u) {       /* inf / nan */
        if (xb & 0x007FFFFFu) return xf;             /* nan */
        return (xb >> 31) ? 0.0f : xf;               /* -inf -> 0, +inf */
    }
    if (xf > 89.0f) return s2p_fm_bits2f(0x7F800000u);
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double INV_LN2 = 1.4426950408889634074;
    /* ln2 = LN2_HI + LN2_LO; LN2_HI has 32 significant bits so k*LN2_HI is
     * exact for |k| < 2^21. */
    const double LN2_HI = 6.93147180369123816490e-01; /* 0x3FE62E42FEE00000 */
    const double LN2_LO = 1.90821492927058770002e-10;
    double t = x * INV_LN2;
    /* round-half-away to an integer; exact for |t| < 2^52 (truncation of a
     * double, the value a conversion to int64 and back gives in that range) */
    double kd = t >= 0.0 ? __builtin_trunc(t + 0.5) : -__builtin_trunc(0.5 - t);
    const int k = (int)kd;
    const double r = (x - kd * LN2_HI) - kd * LN2_LO;
    /* Taylor series of exp(r), Horner form, degree 13 */
    double p = 1.0 / 6227020800.0;          /* 1/13! */
    p = p * r + 1.0 / 479001600.0;          /* 1/12! */
    p = p * r + 1.0 / 39916800.0;           /* 1/11! */
    p = p * r + 1.0 / 3628800.0;            /* 1/10! */
    p = p * r + 1.0 / 362880.0;             /* 1/9!  */
    p = p * r + 1.0 / 40320.0;              /* 1/8!  */
    p = p * r + 1.0 / 5040.0;               /* 1/7!  */
    p = p * r + 1.0 / 720.0;                /* 1/6!  */
    p = p * r + 1.0 / 120.0;                /* 1/5!  */
    p = p * r + 1.0 / 24.0;                 /* 1/4!  */
    p = p * r + 1.0 / 6.0;                  /* 1/3!  */
    p = p * r + 0.5;                        /* 1/2!  */
    p = p * r + 1.0;
    p = p * r + 1.0;
    const double scale = s2p_fm_bits2d((uint64_t)(int64_t)(k + 1023) << 52);
    return (float)(p * scale);
}

/* log(x) rounded to float. */
S2P_FM_QUAL float s2p_logf(float xf) {
    S2P_FM_NOCONTRACT
    const uint32_t xb = s2p_fm_f2bits(xf);
    if (xb == 0u || xb == 0x80000000u) return s2p_fm_bits2f(0xFF800000u); /* -inf */
    if (xb & 0x80000000u) return s2p_fm_bits2f(0x7FC00000u);             /* nan */
    if ((xb & 0x7F800000u) == 0x7F800000u) return xf;                     /* inf/nan */
    const double x = (double)xf; /* exact; every float is a normal double */
    const uint64_t b = s2p_fm_d2bits(x);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    double m = s2p_fm_bits2d((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (m > 1.41421356237309504880) {
        m = m * 0.5;
        e = e + 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double z = s * s;
    /* 2*atanh(s) = 2s * sum_{j>=0} z^j/(2j+1), Horner to j = 12 */
    double q = 1.0 / 25.0;
    q = q * z + 1.0 / 23.0;
    q = q * z + 1.0 / 21.0;
    q = q * z + 1.0 / 19.0;
    q = q * z + 1.0 / 17.0;
    q = q * z + 1.0 / 15.0;
    q = q * z + 1.0 / 13.0;
    q = q * z + 1.0 / 11.0;
    q = q * z + 1.0 / 9.0;
    q = q * z + 1.0 / 7.0;
    q = q * z + 1.0 / 5.0;
    q = q * z + 1.0 / 3.0;
    q = q * z + 1.0;
    const double logm = 2.0 * s * q;
    const double LN2_HI = 6.93147180369123816490e-01;
    const double LN2_LO = 1.90821492927058770002e-10;
    const double ed = (double)e;
    return (float)(ed * LN2_HI + (ed * LN2_LO + logm));
}

#endif /* S2P_FMATH_H */
