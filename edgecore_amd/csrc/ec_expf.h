/*
 * expf as the reference computes it: the reference calls glibc's expf
 * (softmax at src/gpt2.c:546/766, SiLU at src/gpt2.c:589), and the int8 path
 * amplifies a last-bit difference in either into different activation codes,
 * so the GPU must reproduce glibc's result bit for bit, not merely a
 * correctly rounded exp.
 *
 * This is glibc's expf algorithm (sysdeps/ieee754/flt-32/e_expf.c, from
 * ARM's optimized-routines, Szabolcs Nagy 2017): x*32/ln2 = k + r, result
 * 2^(k/32) * P(r) with a 32-entry table of 2^(i/32) and a cubic P, all in
 * double, rounded once to float.  The table entries are the doubles nearest
 * 2^(i/32) with i/32 folded out of the exponent field.  The arithmetic uses
 * the fused multiply-adds that glibc's x86-64 FMA build (the variant its ifunc
 * selects on FMA hosts) produces, including r = fma(InvLn2N, x, -kd).  The
 * same source is compiled for the host by tests/c/expf_exhaustive.c and
 * matched against the host libm on all 2^32 inputs.
 *
 * C and C++ (host) and HIP (device) compatible.
 */
#ifndef EC_EXPF_H
#define EC_EXPF_H

#include <stdint.h>
#include <string.h>

#if defined(__HIP__)
#define EC_EXPF_FN __host__ __device__ static inline
#define EC_EXPF_TABLE static __constant__ const
#else
#define EC_EXPF_FN static inline
#define EC_EXPF_TABLE static const
#endif

EC_EXPF_TABLE uint64_t ec_exp2_32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

/* tab: the 32 entries of ec_exp2_32, wherever the caller keeps a copy
 * (kernels stage them in LDS so the lookup does not wait on memory) */
EC_EXPF_FN float ec_expf_tab(float x, const uint64_t *tab)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0; /* / 32^3 */
    const double c1 = 0x1.ebfce50fac4f3p-3 / 1024.0;  /* / 32^2 */
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    /* the main path for every input; glibc's special cases (|x| >= 88, inf,
     * nan) replace its result below by selects, in glibc's order of
     * precedence, so that a wave takes no branch (the main path of inf or
     * nan yields some value, and its table index stays in 0..31) */
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    double s;
    memcpy(&s, &t, 8);
    const double zz = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
    y = y * s;
    float res = (float)y;
    res = x < -0x1.9fe368p6f ? 0.0f : res;           /* underflow */
    res = x > 0x1.62e42ep6f ? __builtin_inff() : res; /* overflow */
    res = abstop >= 0x7f8u ? x + x : res;             /* inf or nan */
    res = ux == 0xff800000u ? 0.0f : res;             /* -inf */
    return res;
}

EC_EXPF_FN float ec_expf_ref(float x) { return ec_expf_tab(x, ec_exp2_32); }

#endif
