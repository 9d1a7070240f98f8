/*
 * CPU check of the guarded quotient the row kernels use for inputs outside the exhaustive bf16 proof
 * (SmoothQuant-scaled rows, fp16 and fp32 activations; quant_store8r<false, ...> in
 * mica_amd/csrc/norm_quant.hip):
 *
 *     s = max(a, 1e-8f) / 127.0f,  r = 1.0f / s          a: the row's absmax of x
 *     v = x * r                                            one rounded product
 *     if |fract(v) - 0.5| <= 2^-13:  v = x / s            (IEEE division, only near a rounding boundary;
 *                                                          fract as v_fract_f32: min(v - floor(v), 1 - 2^-24))
 *
 * and, for round-half-even, the shorter form the kernels use there:
 *
 *     k = rint(x * r) of the exact product (one FMA with 1.5 * 2^23)
 *     if fract(fma(x, r, 0.5 + 2^-13)) < 2^-12:  k = rint(x / s)
 *
 * The claim: rint(v) == rint(x / s) and trunc(v +- 0.5) == trunc(x / s +- 0.5) for every finite x with
 * |x| <= a.  It holds if |v_fast - x / s| stays far below the 2^-13 window (analytically |v - x / s| <=
 * |x / s| 2^-24 + ulp(v) / 2 < 2^-16 for |x / s| <= 127.5), so this program samples 2^28 (x, a) pairs
 * (x = a bf16 value times a factor in [1e-4, 1e4], the SmoothQuant clamp range, a >= |x| drawn around
 * it), checks the claim on every one, and reports the largest gap between the fast and the IEEE
 * quotient in units of the last place, and how often the slow path runs.
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off guarded_quotient_check.c -o guarded_quotient_check -lm
 * Output: "samples=<n> mismatch_even=<k> mismatch_away=<k> mismatch_fma=<k> max_gap_ulp=<g>
 * slow_fraction=<f> slow_fraction_fma=<f>"; exit status 0 iff every mismatch count is 0 and max_gap_ulp <= 4.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static uint64_t mix(uint64_t z) { /* splitmix64 */
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static float bf16(uint32_t h) {
    uint32_t u = h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static float ulp(float q) {
    int e;
    frexpf(fabsf(q) > 0 ? q : 1e-30f, &e);
    return ldexpf(1.0f, e - 24);
}

int main(void) {
    const long long n = 1ll << 28;
    long long bad_even = 0, bad_away = 0, slow = 0, bad_fma = 0, slow_fma = 0;
    double max_gap = 0.0;
#pragma omp parallel for reduction(+ : bad_even, bad_away, slow, bad_fma, slow_fma) reduction(max : max_gap) schedule(static)
    for (long long i = 0; i < n; ++i) {
        const uint64_t z = mix((uint64_t)i);
        const float xb = bf16((uint32_t)(z & 0x7fff) % 0x7f00u + 0x0080u);              /* normal bf16 */
        const float f = expf(((float)((z >> 16) & 0xffffff) / 16777216.0f) * 18.42f - 9.21f); /* 1e-4 .. 1e4 */
        const float x = ((z >> 40) & 1 ? -1.0f : 1.0f) * (xb * f);
        if (!isfinite(x)) continue;
        const float grow = 1.0f + (float)((z >> 41) & 0xffff) / 65536.0f * ((z >> 57) & 1 ? 0.0f : 3.0f);
        const float a = fabsf(x) * grow;                       /* the absmax: >= |x|, sometimes == |x| */
        if (!isfinite(a)) continue;
        const float s = fmaxf(a, 1e-8f) / 127.0f;
        const float r = 1.0f / s;
        const float q = x / s;
        float v = x * r;
        const double gap = fabs((double)v - (double)q) / ulp(q);
        if (gap > max_gap) max_gap = gap;
        const float fr = fminf(v - floorf(v), 0x1.fffffep-1f);
        if (fabsf(fr - 0.5f) <= 0x1p-13f) {
            v = x / s;
            slow++;
        }
        if (rintf(v) != rintf(q)) bad_even++;
        /* the one-FMA form (round half even) */
        float k = fmaf(x, r, 12582912.0f) - 12582912.0f;
        const float u = fmaf(x, r, 0.5f + 0x1p-13f);
        if (fminf(u - floorf(u), 0x1.fffffep-1f) < 0x1p-12f) {
            k = rintf(x / s);
            slow_fma++;
        }
        if (k != rintf(q)) bad_fma++;
        if (truncf(v >= 0.0f ? v + 0.5f : v - 0.5f) != truncf(q >= 0.0f ? q + 0.5f : q - 0.5f)) bad_away++;
    }
    printf("samples=%lld mismatch_even=%lld mismatch_away=%lld mismatch_fma=%lld max_gap_ulp=%.3f slow_fraction=%.2e "
           "slow_fraction_fma=%.2e\n", n, bad_even, bad_away, bad_fma, max_gap, (double)slow / (double)n,
           (double)slow_fma / (double)n);
    return (bad_even == 0 && bad_away == 0 && bad_fma == 0 && max_gap <= 4.0) ? 0 : 1;
}
