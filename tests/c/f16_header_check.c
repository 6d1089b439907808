/* Compares the host fp16 conversions of include/edgecore.h (used by the
 * synthetic generator) with the F16C instruction of the host CPU: every
 * fp32 bit pattern for f32_to_fp16, every fp16 pattern for fp16_to_f32. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "edgecore.h"

int main(void)
{
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = 0; i < (1ll << 32); i++) {
        uint32_t b = (uint32_t)i;
        float f;
        memcpy(&f, &b, 4);
        uint16_t ref = (uint16_t)_mm_extract_epi16(_mm_cvtps_ph(_mm_set_ss(f), 0), 0);
        if (ref != f32_to_fp16(f)) bad++;
    }
    for (uint32_t h = 0; h < 65536u; h++) {
        float ref = _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128((int)h)));
        float got = fp16_to_f32((uint16_t)h);
        if (isnan(ref) && isnan(got)) continue;
        if (memcmp(&ref, &got, 4)) bad++;
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
