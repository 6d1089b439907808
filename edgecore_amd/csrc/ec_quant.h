/*
 * int8 activation quantization of the reference linear() (src/gpt2.c:446-461):
 *
 *     s = maxa > 0 ? maxa / 127.0f : 1.0f;  q = clamp(lrintf(a / s), -128, 127)
 *
 * ec_quant1 is that formula with the IEEE division.  ec_quant1_rcp gives the
 * same code without a division per element: with r = RN(1/s) (one division per
 * row), y = RN(a*r) is within one ulp of a/s, the remainder a - s*y is exact
 * in one FMA, and y + (a - s*y)*r rounded to nearest is the correctly rounded
 * quotient RN(a/s) (P. Markstein, "Computation of elementary functions on the
 * IBM RISC System/6000 processor", IBM J. R&D 34(1), 1990).  That needs s,
 * 1/s and the quotient away from overflow and underflow: callers take it only
 * for rows whose scale lies in [2^-100, 2^100], where a tiny quotient rounds
 * to code 0 either way.  tests/c/quant_rcp_check.c compares both forms around
 * every half-integer quotient on a sweep of scales.
 *
 * lrintf of NaN or of a magnitude >= 2^63 returns LONG_MIN on x86-64, which
 * clamps to -128; every other value rounds half to even and clamps.
 *
 * C (host) and HIP (device) compatible.
 */
#ifndef EC_QUANT_H
#define EC_QUANT_H

#include <stdint.h>

#if defined(__HIP__)
#define EC_QFN __host__ __device__ static inline
#define EC_QFMA(a, b, c) __builtin_fmaf(a, b, c)
#define EC_QRINT(x) __builtin_rintf(x)
#else
#include <math.h>
#define EC_QFN static inline
#define EC_QFMA(a, b, c) fmaf(a, b, c)
#define EC_QRINT(x) rintf(x)
#endif

EC_QFN int8_t ec_quant_code(float r)
{
    if (!(fabsf(r) < 9.2233720368547758e18f)) return (int8_t)-128;
    return (int8_t)(int)fminf(fmaxf(r, -128.0f), 127.0f);
}

/* the reference formula, IEEE division */
EC_QFN int8_t ec_quant1(float a, float s)
{
    return ec_quant_code(EC_QRINT(a / s));
}

/* rows whose scale s allows ec_quant1_rcp */
EC_QFN int ec_quant_rcp_ok(float s)
{
    return s >= 0x1p-100f && s <= 0x1p100f;
}

/* ec_quant1(a, s) for s with ec_quant_rcp_ok(s), given rcp = 1.0f / s */
EC_QFN int8_t ec_quant1_rcp(float a, float s, float rcp)
{
    const float y = a * rcp;
    const float e = EC_QFMA(-s, y, a);
    const float q = EC_QFMA(e, rcp, y);
    return ec_quant_code(EC_QRINT(q));
}

#endif
