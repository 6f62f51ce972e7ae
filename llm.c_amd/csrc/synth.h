/*
 * synth.h — deterministic synthetic-tensor generator shared by host C and HIP.
 *
 * Every element is a pure function of (seed, stream, index): a splitmix64
 * counter hash gives two uniforms, Box–Muller turns them into one N(0,1)
 * sample, and the result is scaled to N(mean, std) and rounded to float.
 *
 * log, cos and sqrt are written here with + - * / on doubles only (no libm,
 * no fused multiply-add), so the CPU and any GPU produce identical bits: IEEE
 * double + - * / are correctly rounded everywhere.  Accuracy of the helpers
 * is ~1e-15 relative, far below the float rounding of the final sample.
 *
 * Include with contraction disabled (-ffp-contract=off for gcc; the clang
 * pragma below covers hipcc).
 */
#ifndef MOE_SYNTH_H
#define MOE_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define SYNTH_FN static __host__ __device__ inline
#else
#define SYNTH_FN static inline
#endif

#if defined(__clang__)
#define SYNTH_NOCONTRACT _Pragma("clang fp contract(off)")
#else
#define SYNTH_NOCONTRACT
#endif

SYNTH_FN uint64_t synth_mix64(uint64_t z) {
    z ^= z >> 30; z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27; z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}

SYNTH_FN double synth_bits_to_double(uint64_t b) {
    union { uint64_t u; double d; } v; v.u = b; return v.d;
}
SYNTH_FN uint64_t synth_double_to_bits(double d) {
    union { uint64_t u; double d; } v; v.d = d; return v.u;
}

/* Natural log for u in (0, 1]: u = m * 2^e with m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(s), s = (m-1)/(m+1), |s| <= 0.1716, odd series to s^21. */
SYNTH_FN double synth_log(double u) {
    SYNTH_NOCONTRACT
    uint64_t b = synth_double_to_bits(u);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = synth_bits_to_double((b & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL);
    if (m > 1.4142135623730951) { m = m * 0.5; e = e + 1; }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    return 2.0 * s * p + (double)e * 0.6931471805599453;
}

/* sqrt(y) for y > 0 by Newton's method from an exponent-halved start. */
SYNTH_FN double synth_sqrt(double y) {
    SYNTH_NOCONTRACT
    uint64_t b = synth_double_to_bits(y);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double x = synth_bits_to_double((uint64_t)((e / 2) + 1023) << 52);
    for (int i = 0; i < 8; ++i) x = 0.5 * (x + y / x);
    return x;
}

/* cos(2*pi*u) for u in [0, 1): quadrant split, Taylor series on [0, pi/2). */
SYNTH_FN double synth_cos2pi(double u) {
    SYNTH_NOCONTRACT
    double v = u * 4.0;
    int q = (int)v;               /* 0..3 */
    if (q > 3) q = 3;
    double f = (v - (double)q) * 1.5707963267948966;   /* [0, pi/2) */
    double f2 = f * f;
    /* cos f and sin f, Horner in f^2 to degree 20 / 21. */
    double c = 1.0 / 2432902008176640000.0;              /* 1/20! */
    c = -c * f2 + 1.0 / 6402373705728000.0;             /* 1/18! */
    c = -c * f2 + 1.0 / 20922789888000.0;               /* 1/16! */
    c = -c * f2 + 1.0 / 87178291200.0;                  /* 1/14! */
    c = -c * f2 + 1.0 / 479001600.0;                    /* 1/12! */
    c = -c * f2 + 1.0 / 3628800.0;                      /* 1/10! */
    c = -c * f2 + 1.0 / 40320.0;                        /* 1/8!  */
    c = -c * f2 + 1.0 / 720.0;                          /* 1/6!  */
    c = -c * f2 + 1.0 / 24.0;                           /* 1/4!  */
    c = -c * f2 + 0.5;                                  /* 1/2!  */
    c = -c * f2 + 1.0;
    double s = 1.0 / 51090942171709440000.0;            /* 1/21! */
    s = -s * f2 + 1.0 / 121645100408832000.0;           /* 1/19! */
    s = -s * f2 + 1.0 / 355687428096000.0;              /* 1/17! */
    s = -s * f2 + 1.0 / 1307674368000.0;                /* 1/15! */
    s = -s * f2 + 1.0 / 6227020800.0;                   /* 1/13! */
    s = -s * f2 + 1.0 / 39916800.0;                     /* 1/11! */
    s = -s * f2 + 1.0 / 362880.0;                       /* 1/9!  */
    s = -s * f2 + 1.0 / 5040.0;                         /* 1/7!  */
    s = -s * f2 + 1.0 / 120.0;                          /* 1/5!  */
    s = -s * f2 + 1.0 / 6.0;                            /* 1/3!  */
    s = (-s * f2 + 1.0) * f;
    if (q == 0) return c;
    if (q == 1) return -s;
    if (q == 2) return -c;
    return s;
}

/* One N(mean, std) sample for element `idx` of tensor `stream`. */
SYNTH_FN float synth_normal(uint64_t seed, uint64_t stream, uint64_t idx,
                            float mean, float std) {
    SYNTH_NOCONTRACT
    uint64_t key = synth_mix64(seed * 0x9e3779b97f4a7c15ULL + 0x632be59bd9b4e019ULL)
                 ^ synth_mix64(stream + 0xd1b54a32d192ed03ULL);
    uint64_t h1 = synth_mix64(key + (2 * idx + 1) * 0x9e3779b97f4a7c15ULL);
    uint64_t h2 = synth_mix64(key + (2 * idx + 2) * 0x9e3779b97f4a7c15ULL);
    double u1 = (double)((h1 >> 11) + 1) * (1.0 / 9007199254740992.0);  /* (0,1] */
    double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);        /* [0,1) */
    double r = synth_sqrt(-2.0 * synth_log(u1));
    if (u1 == 1.0) r = 0.0;
    double z = r * synth_cos2pi(u2);
    return (float)((double)mean + (double)std * z);
}

/* Uniform integer in [0, n) for element `idx` of tensor `stream`. */
SYNTH_FN uint32_t synth_uniform_int(uint64_t seed, uint64_t stream, uint64_t idx,
                                    uint32_t n) {
    uint64_t key = synth_mix64(seed * 0x9e3779b97f4a7c15ULL + 0x632be59bd9b4e019ULL)
                 ^ synth_mix64(stream + 0xd1b54a32d192ed03ULL);
    uint64_t h = synth_mix64(key + (idx + 1) * 0x9e3779b97f4a7c15ULL);
    return (uint32_t)(((h >> 32) * (uint64_t)n) >> 32);
}

#endif /* MOE_SYNTH_H */
