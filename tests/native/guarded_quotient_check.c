/*
 * CPU check of the guarded quotient the row kernels use for inputs outside the exhaustive bf16 proof
 * (SmoothQuant-scaled rows, fp16 and fp32 activations; quant_store8r<false, ...> in
 * mica_amd/csrc/norm_quant.hip), with the tie window W = 2^-15:
 *
 *     s = max(a, 1e-8f) / 127.0f,  r = 1.0f / s          a: the row's absmax of x
 *     v = x * r                                            one rounded product
 *     if |fract(v) - 0.5| <= W:  v = x / s                (IEEE division, only near a rounding boundary;
 *                                                          fract as v_fract_f32: min(v - floor(v), 1 - 2^-24))
 *
 * and, for round-half-even, the shorter form the kernels use there:
 *
 *     k = rint(x * r) of the exact product (one FMA with 1.5 * 2^23)
 *     if fract(fma(x, r, 0.5 + W)) < 2 W:  k = rint(x / s)
 *
 * The claim: rint(v) == rint(x / s), trunc(v +- 0.5) == trunc(x / s +- 0.5) and k == rint(x / s) for
 * every finite x with |x / s| <= 127.5.  Analytically v, the exact x r and RN(x / s) lie within 2^-16 of
 * each other there, so the results can only differ within 2^-16 of a boundary j + 0.5, which the guard
 * covers.  Two checks:
 *
 *   1. 2^28 random (x, a) pairs: x a bf16 value times a factor in [1e-4, 1e4] (the SmoothQuant clamp
 *      range), a >= |x| drawn around it; also the largest gap between v and the IEEE quotient in ulps.
 *   2. The boundaries themselves: everything is invariant under scaling x and s by one power of two
 *      (no subnormals involved), so s in [1, 2) stands for every normal scale.  For 2^15 values of s
 *      spread over [1, 2) (mantissa high bits stepped, low bits scrambled, plus 1 and 2 - 2^-23), every
 *      boundary j + 0.5 (j = -128 .. 127) and every fp32 x whose x / s lies within 2 W of it (both
 *      sides), check all three claims.  "hazards" counts the x where the unguarded product's integer
 *      differs from the IEEE quotient's: the cases the guard exists for.
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off guarded_quotient_check.c -o guarded_quotient_check -lm
 * Output: "samples=<n> mismatch_even=<k> mismatch_away=<k> mismatch_fma=<k> max_gap_ulp=<g>
 * slow_fraction=<f> slow_fraction_fma=<f> sweep_scales=<n> sweep_values=<n> sweep_mismatch=<k>
 * sweep_hazards=<k> sweep_hazards_fma=<k>"; exit status 0 iff every mismatch count is 0 and
 * max_gap_ulp <= 4.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#ifndef WINDOW /* the kernels' kTieWindow; a build with a smaller one shows that the sweep finds mismatches */
#define WINDOW 0x1p-15f
#endif

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
static float fract(float v) { return fminf(v - floorf(v), 0x1.fffffep-1f); }
static float away(float v) { return truncf(v >= 0.0f ? v + 0.5f : v - 0.5f); }

/* the three kernel forms for one (x, s): bit 0 = half even, bit 1 = half away, bit 2 = the FMA form,
   set where the form's integer differs from the IEEE quotient's */
static int check(float x, float s, float r, long long *slow, long long *slow_fma) {
    const float q = x / s;
    float v = x * r;
    if (fabsf(fract(v) - 0.5f) <= WINDOW) {
        v = x / s;
        ++*slow;
    }
    float k = fmaf(x, r, 12582912.0f) - 12582912.0f;
    if (fract(fmaf(x, r, 0.5f + WINDOW)) < 2.0f * WINDOW) {
        k = rintf(x / s);
        ++*slow_fma;
    }
    return (rintf(v) != rintf(q)) | ((away(v) != away(q)) << 1) | ((k != rintf(q)) << 2);
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
        const double gap = fabs((double)(x * r) - (double)q) / ulp(q);
        if (gap > max_gap) max_gap = gap;
        const int bad = check(x, s, r, &slow, &slow_fma);
        bad_even += bad & 1;
        bad_away += (bad >> 1) & 1;
        bad_fma += (bad >> 2) & 1;
    }

    /* 2: every x around every boundary, 2^15 scales */
    const int n_scales = 1 << 15;
    long long values = 0, sweep_bad = 0, hazards = 0, hazards_fma = 0, sweep_slow = 0, sweep_slow_fma = 0;
#pragma omp parallel for reduction(+ : values, sweep_bad, hazards, hazards_fma, sweep_slow, sweep_slow_fma) schedule(dynamic, 64)
    for (int i = 0; i < n_scales; ++i) {
        uint32_t mant = ((uint32_t)i << 8) | (uint32_t)(mix(0x5eedull + (uint64_t)i) & 0xff);
        if (i == 0) mant = 0;                      /* s = 1 */
        if (i == n_scales - 1) mant = 0x7fffff;    /* s = 2 - 2^-23 */
        const uint32_t bits = 0x3f800000u | mant;
        float s;
        memcpy(&s, &bits, 4);
        const float r = 1.0f / s;
        for (int j = -128; j <= 127; ++j) {
            const double t = (double)j + 0.5;      /* the boundary j + 0.5 */
            const double lo = (t - 2.0 * WINDOW) * s, hi = (t + 2.0 * WINDOW) * s;
            float x = nextafterf((float)lo, -INFINITY);
            const float end = nextafterf((float)hi, INFINITY);
            for (; x <= end; x = nextafterf(x, INFINITY)) {
                if (fabs((double)x / (double)s) > 127.5) continue;
                ++values;
                const int bad = check(x, s, r, &sweep_slow, &sweep_slow_fma);
                sweep_bad += bad != 0;
                hazards += rintf(x * r) != rintf(x / s);
                hazards_fma += (fmaf(x, r, 12582912.0f) - 12582912.0f) != rintf(x / s);
            }
        }
    }
    printf("samples=%lld mismatch_even=%lld mismatch_away=%lld mismatch_fma=%lld max_gap_ulp=%.3f slow_fraction=%.2e "
           "slow_fraction_fma=%.2e sweep_scales=%d sweep_values=%lld sweep_mismatch=%lld sweep_hazards=%lld "
           "sweep_hazards_fma=%lld\n", n, bad_even, bad_away, bad_fma, max_gap, (double)slow / (double)n,
           (double)slow_fma / (double)n, n_scales, values, sweep_bad, hazards, hazards_fma);
    return (bad_even == 0 && bad_away == 0 && bad_fma == 0 && sweep_bad == 0 && max_gap <= 4.0) ? 0 : 1;
}
