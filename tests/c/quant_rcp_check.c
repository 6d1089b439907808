/*
 * ec_quant1_rcp (reciprocal + one Markstein correction) against the IEEE
 * division form ec_quant1 of the reference quantizer, on the inputs where a
 * difference could show: quotients within 64 ulps of every half-integer in
 * [-128.5, 128.5] (ties included), for a sweep of row scales s = maxa / 127
 * (every binade of maxa from 2^-90 to 2^90, mantissas at both ends and
 * random), plus random activations and the rows' extremes +-maxa.  Also
 * compares the full quotient RN(a/s) itself.  Prints the number of checked
 * pairs and exits 1 on the first mismatch.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -I edgecore_amd/csrc quant_rcp_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "ec_quant.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next(void)
{
    uint64_t z = (rng += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static long long checked = 0;

static int check(float a, float s, float rcp)
{
    checked++;
    const float y = a * rcp;
    const float e = fmaf(-s, y, a);
    const float q = fmaf(e, rcp, y);
    const float qd = a / s;
    /* the quotient itself must agree where it can round to a non-zero code
       (below 2^-20 both forms give code 0; a subnormal a may then leave the
       remainder inexact) */
    if (fabsf(qd) >= 0x1p-20f && bits(q) != bits(qd) && !(isnan(q) && isnan(qd))) {
        printf("quotient mismatch: a=%a s=%a rcp=%a: rcp path %a, division %a\n", a, s, rcp, q, qd);
        return 1;
    }
    if (ec_quant1_rcp(a, s, rcp) != ec_quant1(a, s)) {
        printf("code mismatch: a=%a s=%a\n", a, s);
        return 1;
    }
    return 0;
}

static int check_scale(float maxa)
{
    const float s = maxa > 0.0f ? maxa / 127.0f : 1.0f;
    if (!ec_quant_rcp_ok(s)) return 0;
    const float rcp = 1.0f / s;
    if (check(maxa, s, rcp) || check(-maxa, s, rcp)) return 1;
    for (int h = -257; h <= 257; h++) {  /* quotient h/2 */
        const float c = (float)((double)h * 0.5 * (double)s);
        const uint32_t cb = bits(c);
        for (int d = -64; d <= 64; d++) {
            const float a = from_bits((uint32_t)((int32_t)cb + d));
            if (fabsf(a) > maxa * 1.0001f) continue;
            if (check(a, s, rcp)) return 1;
        }
    }
    for (int i = 0; i < 2000; i++) {
        const float u = (float)((double)(next() >> 11) * 0x1p-53 * 2.0 - 1.0);
        if (check(u * maxa, s, rcp)) return 1;
    }
    return 0;
}

int main(void)
{
    for (int ex = -90; ex <= 90; ex++) {
        const float lo = ldexpf(1.0f, ex), hi = nextafterf(ldexpf(1.0f, ex + 1), 0.0f);
        if (check_scale(lo) || check_scale(hi)) return 1;
        for (int i = 0; i < 24; i++) {
            const float m = from_bits((bits(lo) & 0xFF800000u) | (uint32_t)(next() & 0x7FFFFFu));
            if (check_scale(m)) return 1;
        }
    }
    printf("ec_quant1_rcp == ec_quant1 on %lld (activation, scale) pairs\n", checked);
    return 0;
}
