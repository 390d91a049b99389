/* Exhaustive check of the division-free quant step (test infrastructure).
 *
 * The bf16 quant kernels compute q = clamp(rint(v / s), +-127) as
 *   rs = 1 / s;  q0 = v * rs;  r = fma(-q0, s, v);  q1 = fma(r, rs, q0);  q = clamp(rint(q1), +-127)
 * This program compares rint(q1) with rint(v / s) (IEEE binary32, round to nearest even) for every
 * positive finite bf16 absmax a, s = max(a, 1e-8) / 127, and every bf16 v with |v| <= a, and also
 * counts how often the uncorrected rint(v * rs) differs.  Output: "pairs P mismatches Q plain R". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int main(void) {
    long long pairs = 0, bad = 0, plain = 0;
#pragma omp parallel for reduction(+ : pairs, bad, plain) schedule(dynamic, 64)
    for (int ah = 0; ah < 0x7f80; ++ah) {
        const float a = bf((uint16_t)ah);
        const float s = fmaxf(a, 1e-8f) / 127.0f;
        const float rs = 1.0f / s;
        for (int vh = 0; vh < 0x10000; ++vh) {
            const float v = bf((uint16_t)vh);
            if (!(fabsf(v) <= a)) continue;
            const float q = rintf(v / s);
            const float q0 = v * rs;
            const float q1 = fmaf(fmaf(-q0, s, v), rs, q0);
            ++pairs;
            bad += rintf(q1) != q;
            plain += rintf(q0) != q;
        }
    }
    printf("pairs %lld mismatches %lld plain %lld\n", pairs, bad, plain);
    return 0;
}
