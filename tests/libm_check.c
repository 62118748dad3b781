/* libm_check.c - compares the package's restated expf/log1pf (dsv4_libm.h,
 * the source the GPU kernels compile) with the host libm, bit for bit.
 * Usage: libm_check STRIDE  (1 = every input; the test suite uses a stride).
 * Prints "<fn> <checked> <mismatches>" lines; exit status 1 on any mismatch.
 * Built with -ffp-contract=off so that only the explicit fma() calls fuse. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

#include "dsv4_libm.h"

int main(int argc, char **argv)
{
    const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
    long n = 0, bad = 0;
    /* expf on every float up to the overflow / underflow thresholds and past
     * them, both signs */
    for (uint64_t u = 0; u < 0x80000000ull; u += stride) {
        for (int s = 0; s < 2; s++) {
            float x = dsv4_libm_u2f((uint32_t)u | (s ? 0x80000000u : 0u));
            if (!(fabsf(x) <= 120.0f)) continue;
            float a = expf(x), b = dsv4_libm_expf(x);
            n++;
            if (dsv4_libm_f2u(a) != dsv4_libm_f2u(b)) {
                if (bad < 5) printf("  expf mismatch x=%a libm=%a restated=%a\n", x, a, b);
                bad++;
            }
        }
    }
    printf("expf %ld %ld\n", n, bad);
    long n2 = 0, bad2 = 0;
    for (uint64_t u = 0; u <= 0x7f800000ull; u += stride) {
        float x = dsv4_libm_u2f((uint32_t)u);
        float a = log1pf(x), b = dsv4_libm_log1pf_nonneg(x);
        n2++;
        if (dsv4_libm_f2u(a) != dsv4_libm_f2u(b)) {
            if (bad2 < 5) printf("  log1pf mismatch x=%a libm=%a restated=%a\n", x, a, b);
            bad2++;
        }
    }
    printf("log1pf %ld %ld\n", n2, bad2);
    return (bad || bad2) ? 1 : 0;
}
