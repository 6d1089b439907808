/* Compares ec_expf_ref (edgecore_amd/csrc/ec_expf.h, the expf the GPU
 * kernels use) with the host libm's expf over the input bit patterns
 * [lo, hi).  Prints the mismatch count and the first few mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ec_expf.h"

int main(int argc, char **argv)
{
    uint64_t lo = argc > 1 ? strtoull(argv[1], NULL, 0) : 0;
    uint64_t hi = argc > 2 ? strtoull(argv[2], NULL, 0) : (1ull << 32);
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = (int64_t)lo; i < (int64_t)hi; i++) {
        uint32_t b = (uint32_t)i;
        float x, g, m;
        memcpy(&x, &b, 4);
        g = expf(x);
        m = ec_expf_ref(x);
        if (isnan(g) && isnan(m)) continue;
        if (memcmp(&g, &m, 4) != 0) {
            bad++;
            if (bad < 4) printf("x=%a glibc=%a ec=%a\n", x, g, m);
        }
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
