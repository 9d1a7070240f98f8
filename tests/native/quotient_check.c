/*
 * Exhaustive proof, on the CPU, of the quotient the gfx950 quantizer kernels use for bf16 inputs
 * (quant_store8r<true, ...> in mica_amd/csrc/norm_quant.hip):
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
 * It also checks the unclamped half-even path of the row kernels (quant_store8r in
 * mica_amd/csrc/norm_quant.hip): the int8 taken as the low byte of the bits of v + 12582912.0f
 * equals clamp(rint(x / s), -127, 127) for every pair, and |v| never reaches 127.5 (so the clamp the
 * reference applies never changes a finite row's result).
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off quotient_check.c -o quotient_check -lm
 * Output: "pairs=<n> mismatch_even=<k> mismatch_away=<k> mismatch_magic=<k> max_abs_v=<f>";
 * exit status 0 iff all mismatch counts are 0 and max_abs_v < 127.5.
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
    long long pairs = 0, bad_even = 0, bad_away = 0, bad_magic = 0;
    float max_abs_v = 0.0f;
#pragma omp parallel for reduction(+ : pairs, bad_even, bad_away, bad_magic) reduction(max : max_abs_v) schedule(dynamic, 64)
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
                /* the row kernels' half-even int8: low byte of v + 1.5 * 2^23, no clamp */
                const float m = v + 12582912.0f;
                uint32_t mb;
                memcpy(&mb, &m, 4);
                const int8_t got = (int8_t)(mb & 0xffu);
                const float ref = fminf(fmaxf(rintf(q), -127.0f), 127.0f);
                if ((int)got != (int)ref) bad_magic++;
                if (fabsf(v) > max_abs_v) max_abs_v = fabsf(v);
                pairs++;
            }
        }
    }
    printf("pairs=%lld mismatch_even=%lld mismatch_away=%lld mismatch_magic=%lld max_abs_v=%.7f\n", pairs, bad_even,
           bad_away, bad_magic, max_abs_v);
    return (bad_even == 0 && bad_away == 0 && bad_magic == 0 && max_abs_v < 127.5f) ? 0 : 1;
}
