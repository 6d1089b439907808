/* The fp32 -> bfloat16 packers against the definition, on all 2^32 inputs.
 *
 * Checked: ec_f32_to_bf16 (edgecore_amd/csrc/ecm.c, the generator's) and
 * or_f32_to_bf16 (oracle/ec_oracle.c), both restating edgecore/ecm.py:27-41.
 * The definition used here is IEEE round-to-nearest-even written as a
 * distance comparison, not the bias-and-shift of the restatements: the two
 * bf16 neighbours of x (truncation and one step away from zero) are widened
 * to double, the nearer one wins, a tie goes to the even significand, and a
 * value past the largest finite bf16 compares against 2^128 (the exponent
 * taken as unbounded), so it overflows to infinity exactly at the halfway
 * point.  Every NaN maps to 0x7fc0 (ecm.py's nan_mask). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint16_t ec_f32_to_bf16(float f);
uint16_t or_f32_to_bf16(float f);

static double bf16_value(uint16_t b)
{
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return (double)f;
}

static uint16_t nearest_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if (isnan(f)) return 0x7fc0u;
    const uint16_t lo = (uint16_t)(x >> 16);
    if ((x & 0xffffu) == 0) return lo; /* representable (incl. +-inf, +-0) */
    const uint16_t hi = (uint16_t)(lo + 1u); /* one step away from zero */
    const double v = fabs((double)f);
    const double vlo = fabs(bf16_value(lo));
    const double vhi = (hi & 0x7fffu) == 0x7f80u ? ldexp(1.0, 128) : fabs(bf16_value(hi));
    const double dlo = v - vlo, dhi = vhi - v;
    if (dlo < dhi) return lo;
    if (dhi < dlo) return hi;
    return (lo & 1u) ? hi : lo;
}

int main(void)
{
    unsigned long long bad_ec = 0, bad_or = 0;
#pragma omp parallel for reduction(+ : bad_ec, bad_or) schedule(static)
    for (long long i = 0; i <= 0xffffffffLL; i++) {
        const uint32_t x = (uint32_t)i;
        float f;
        memcpy(&f, &x, 4);
        const uint16_t want = nearest_bf16(f);
        if (ec_f32_to_bf16(f) != want) bad_ec++;
        if (or_f32_to_bf16(f) != want) bad_or++;
    }
    printf("ec_f32_to_bf16 mismatches %llu, or_f32_to_bf16 mismatches %llu\n", bad_ec, bad_or);
    return (bad_ec || bad_or) ? 1 : 0;
}
