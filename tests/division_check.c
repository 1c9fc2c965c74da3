/* Checks the quotient identity the beam kernel relies on (stlq_amd/csrc/k_beam.hip, QuotFast):
 * for d in [2^-20, 2^20] and |s| in [2^-100, 2^100], with y = RN(1/d),
 *     q0 = RN(s*y),  r = fma(d, q0, -s),  q = fma(-r, y, q0)
 * equals the IEEE quotient RN(s/d) bit for bit (Markstein's correction with a correctly rounded
 * reciprocal). Part 1 runs every numerator mantissa against divisor mantissas with edge
 * patterns (all ones, single bits, runs) and random ones, at several exponent pairs; part 2
 * samples the whole guarded exponent range. Prints the mismatch count; exit status 1 if any.
 * Build: gcc -O2 -mfma -ffp-contract=off -fopenmp division_check.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float quot(float s, float d, float y) {
    float q0 = s * y;
    float r = fmaf(d, q0, -s);
    return fmaf(-r, y, q0);
}

int main(int argc, char** argv) {
    int nd = argc > 1 ? atoi(argv[1]) : 64;
    long nsamp = argc > 2 ? atol(argv[2]) : 50000000L;
    long bad = 0, checked = 0;
    const int dexp[3] = {-20, 0, 19};
    const int sexp[2] = {0, 1};
#pragma omp parallel for reduction(+ : bad, checked) schedule(dynamic, 1)
    for (int i = 0; i < nd; ++i) {
        uint32_t m;
        if (i == 0) m = 0x7FFFFF;
        else if (i == 1) m = 0;
        else if (i < 24) m = 0x7FFFFF ^ (1u << (i - 1));
        else if (i < 46) m = 1u << (i - 24);
        else {
            uint64_t z = 0x9E3779B97F4A7C15ULL * (uint64_t)(i + 1);
            z ^= z >> 29; z *= 0xBF58476D1CE4E5B9ULL; z ^= z >> 32;
            m = (uint32_t)z & 0x7FFFFF;
        }
        for (int a = 0; a < 3; ++a) {
            float d = bf(((uint32_t)(dexp[a] + 127) << 23) | m);
            float y = 1.0f / d;
            for (int b = 0; b < 2; ++b) {
                for (uint32_t ms = 0; ms < 0x800000u; ++ms) {
                    float s = bf(((uint32_t)(sexp[b] + 127) << 23) | ms);
                    bad += fb(quot(s, d, y)) != fb(s / d);
                    bad += fb(quot(-s, d, y)) != fb(-s / d);
                    checked += 2;
                }
            }
        }
    }
    uint64_t st = 0x1234567ULL;
    for (long i = 0; i < nsamp; ++i) {
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        uint32_t md = (uint32_t)(st >> 41) & 0x7FFFFF;
        int de = (int)((st >> 20) % 41) - 20;
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        uint32_t ms = (uint32_t)(st >> 41) & 0x7FFFFF;
        int se = (int)((st >> 20) % 200) - 100;
        float d = bf(((uint32_t)(de + 127) << 23) | md);
        float s = bf(((uint32_t)(se + 127) << 23) | ms | ((st >> 63) ? 0x80000000u : 0u));
        if (d > 0x1p20f) continue;
        bad += fb(quot(s, d, 1.0f / d)) != fb(s / d);
        checked++;
    }
    printf("checked=%ld mismatches=%ld\n", checked, bad);
    return bad != 0;
}
