/*
 * Exhaustive proof, on the CPU, of the quotient the gfx950 quantizer kernels use for bf16 inputs
 * (quantize_one<true> in mica_amd/csrc/common.h):
 *
 *     s   = max(a, 1e-8f) / 127.0f           a: the row's absmax, a bf16 value >= |x|
 *     inv = 1.0f / s                         (once per row, IEEE division)
 *     y   = x * inv;  rem = fmaf(-y, s, x);  v = fmaf(rem, inv, y)
 *
 * For every finite bf16 x and every positive finite bf16 a with |x| <= a, this checks that
 *     rint(v)                     == rint(x / s)                       (half to even)
 *     trunc(v >= 0 ? v+.5 : v-.5) == trunc(q >= 0 ? q+.5 : q-.5), q = x / s   (half away)
 * where x / s is the IEEE fp32 quotient.  Both sides are then clamped to +-127 identically, so equal
 * pre-clamp values mean equal int8 outputs.  (v itself is not always the correctly rounded quotient;
 * only the rounded integers are claimed equal.)
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off quotient_check.c -o quotient_check -lm
 * Output: "pairs=<n> mismatch_even=<k> mismatch_away=<k>"; exit status 0 iff both are 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16(uint32_t h) {
    uint32_t u = h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int main(void) {
    long long pairs = 0, bad_even = 0, bad_away = 0;
#pragma omp parallel for reduction(+ : pairs, bad_even, bad_away) schedule(dynamic, 64)
    for (uint32_t ab = 1; ab < 0x7f80u; ++ab) { /* positive finite bf16 absmax values */
        const float a = bf16(ab);
        const float s = fmaxf(a, 1e-8f) / 127.0f;
        const float inv = 1.0f / s;
        for (uint32_t xb = 0; xb < 0x7f80u; ++xb) {
            const float xm = bf16(xb);
            if (xm > a) break; /* bf16 magnitudes increase with the bit pattern */
            for (int sign = 0; sign < 2; ++sign) {
                const float x = sign ? -xm : xm;
                const float q = x / s;
                const float y = x * inv;
                const float rem = fmaf(-y, s, x);
                const float v = fmaf(rem, inv, y);
                if (rintf(v) != rintf(q)) bad_even++;
                const float av = truncf(v >= 0.0f ? v + 0.5f : v - 0.5f);
                const float aq = truncf(q >= 0.0f ? q + 0.5f : q - 0.5f);
                if (av != aq) bad_away++;
                pairs++;
            }
        }
    }
    printf("pairs=%lld mismatch_even=%lld mismatch_away=%lld\n", pairs, bad_even, bad_away);
    return (bad_even == 0 && bad_away == 0) ? 0 : 1;
}
