/* Checks the division-free scale used by the RotorQuant kernels,
 *   q0 = RN(m * y), r = fma(-q0, qmax, m), q1 = RN(q0 + r*y) (one fma),
 * with y = RN(1/qmax), against the IEEE quotient m / qmax for every mantissa
 * of the binades whose exponents are given on the command line, for every
 * qmax = 2^(bits-1) - 1, bits in [2, 8]. Prints the number of mismatches.
 * Build: gcc -O2 -ffp-contract=off -mfma markstein_check.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

int main(int argc, char **argv) {
    long checked = 0, bad = 0;
    for (int bits = 2; bits <= 8; ++bits) {
        const float qmax = (float)((1u << (bits - 1)) - 1u);
        const float y = 1.0f / qmax;
        for (int a = 1; a < argc; ++a) {
            const uint32_t e = (uint32_t)atoi(argv[a]);
            for (uint32_t mant = 0; mant < (1u << 23); ++mant) {
                const float m = from_bits((e << 23) | mant);
                const float q0 = m * y;
                const float r = fmaf(-q0, qmax, m);
                const float q1 = r == r ? fmaf(r, y, q0) : q0;
                ++checked;
                if (q1 != m / qmax) ++bad;
            }
        }
    }
    printf("%ld %ld\n", checked, bad);
    return 0;
}
