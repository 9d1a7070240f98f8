/*
 * Exhaustive proof, on the CPU, of the one-FMA half-even quantizer the gfx950 row kernels use for
 * unsmoothed bf16 rows (quant_store8_fma in mica_amd/csrc/norm_quant.hip):
 *
 *     s   = max(a, 1e-8f) / 127.0f           a: the row's absmax, a bf16 value >= |x|
 *     inv = 1.0f / s                         (IEEE division, once per row)
 *     h   = a * 0.5f                         (exact)
 *     qh  = rint(h / s)                      (IEEE division, once per row)
 *     qf  = fmaf(h, inv, 1.5 * 2^23) - 1.5 * 2^23
 *     r   = inv moved one ulp toward qh when qh != qf (once per row)
 *     q   = low byte of the bits of fmaf(x, r, 1.5 * 2^23)     (per element: one FMA)
 *
 * fmaf(x, r, 1.5 * 2^23) rounds the exact product x * r to an integer, half to even, in one step.
 * With r = 1 / s rounded, that integer can only differ from rint(x / s) (the reference's
 * torch.round of the IEEE quotient) where x / s lies next to a half-integer; for bf16 x and a the
 * only such x is a / 2 (quotient 63.5 up to the rounding of s), and moving r one ulp toward the
 * correct side for that x leaves every other x of the row unchanged.  This program checks the
 * claim for every finite bf16 x and every positive finite bf16 a with |x| <= a:
 *
 *     q == clamp(rint(x / s), -127, 127)
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off fma_quotient_check.c -o fma_quotient_check -lm
 * Output: "pairs=<n> mismatch=<k> adjusted_rows=<k>"; exit status 0 iff mismatch == 0.
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

static float step_ulp(float v, int dir) {
    uint32_t b;
    memcpy(&b, &v, 4);
    b += (uint32_t)dir; /* v > 0: +1 is one ulp up, -1 one ulp down */
    memcpy(&v, &b, 4);
    return v;
}

int main(void) {
    const float magic = 12582912.0f;
    long long pairs = 0, bad = 0, adjusted = 0;
#pragma omp parallel for reduction(+ : pairs, bad, adjusted) schedule(dynamic, 64)
    for (uint32_t ab = 1; ab < 0x7f80u; ++ab) { /* positive finite bf16 absmax values */
        const float a = bf16(ab);
        const float s = fmaxf(a, 1e-8f) / 127.0f;
        const float inv = 1.0f / s;
        const float h = a * 0.5f;
        const float qh = rintf(h / s);
        const float qf = fmaf(h, inv, magic) - magic;
        const int dir = qh > qf ? 1 : (qh < qf ? -1 : 0);
        const float r = dir ? step_ulp(inv, dir) : inv;
        adjusted += dir != 0;
        for (uint32_t xb = 0; xb < 0x7f80u; ++xb) {
            const float xm = bf16(xb);
            if (xm > a) break; /* bf16 magnitudes increase with the bit pattern */
            for (int sign = 0; sign < 2; ++sign) {
                const float x = sign ? -xm : xm;
                const float m = fmaf(x, r, magic);
                uint32_t mb;
                memcpy(&mb, &m, 4);
                const int8_t got = (int8_t)(mb & 0xffu);
                const float ref = fminf(fmaxf(rintf(x / s), -127.0f), 127.0f);
                if ((int)got != (int)ref) bad++;
                pairs++;
            }
        }
    }
    printf("pairs=%lld mismatch=%lld adjusted_rows=%lld\n", pairs, bad, adjusted);
    return bad == 0 ? 0 : 1;
}
