/* Exhaustive check of the GPU quantizer's scale formula (device.h q8_scale):
 * for every finite float m >= 0, s0 = m * RN(1/127),
 * s = fma(fma(-s0, 127, m), RN(1/127), s0) must equal the IEEE quotient
 * m / 127 that the reference computes (runq.c:117-139).  Prints the number
 * of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float c = 1.0f / 127.0f;
    unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u < 0x7f800000LL; u++) {
        const uint32_t b = (uint32_t)u;
        float m;
        memcpy(&m, &b, 4);
        const float q = m / 127.0f;
        const float s0 = m * c;
        const float s = fmaf(fmaf(-s0, 127.0f, m), c, s0);
        uint32_t qb, sb;
        memcpy(&qb, &q, 4);
        memcpy(&sb, &s, 4);
        bad += qb != sb;
    }
    printf("%llu\n", bad);
    return 0;
}
