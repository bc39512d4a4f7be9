/* Exhaustive check, on the CPU, of the division forms the GPU's Q8_1
 * quantization uses for a block amax a (q8_scales in
 * hbd-siglip2.cpp_amd/csrc/s2x_device.h): Markstein's division against the
 * IEEE quotients.
 *   d   = a / 127: q0 = a RN(1/127); d = fma(fma(-127, q0, a), RN(1/127), q0)
 *   inv = 127 / a: r0 = either float next to 1 / a (v_rcp_f32 is within
 *         1 ulp); p0 = 127 r0; inv = fma(fma(-a, p0, 127), r0, p0)
 * Prints "d_bad N", "inv_bad N" (every significand of a in [1, 2), both r0)
 * and "inv_exp_bad N" (every exponent from -121 to 126, sampled
 * significands, both r0).  PLANT = 1 and 2 leave out the remainder
 * correction of inv and of d: mistakes the check must see (a reciprocal
 * 1 ulp off is not one: the correction absorbs it). */
#ifndef PLANT
#define PLANT 0
#endif
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float fb(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static void neighbours(float a, float *lo, float *hi) {
    const double r = 1.0 / (double)a; /* 1/a to 53 bits: enough to order the floats around it */
    float f = (float)r;
    if ((double)f == r) { *lo = *hi = f; return; }
    if ((double)f < r) { *lo = f; *hi = nextafterf(f, INFINITY); }
    else { *hi = f; *lo = nextafterf(f, 0.0f); }
}

static float inv_fast(float a, float r0) {
    const float p0 = 127.0f * r0;
    return PLANT == 1 ? p0 : fmaf(fmaf(-a, p0, 127.0f), r0, p0);
}

int main(void) {
    const float r127 = (float)(1.0 / 127.0);
    long d_bad = 0;
    /* (dynamic: the subnormal end is slow on the CPU) */
#pragma omp parallel for schedule(dynamic, 1 << 20) reduction(+ : d_bad)
    for (int64_t u = 1; u < 0x7F800000LL; ++u) { /* every positive finite float */
        const float a = fb((uint32_t)u), q0 = a * r127;
        const float d = PLANT == 2 ? q0 : fmaf(fmaf(-127.0f, q0, a), r127, q0);
        d_bad += bf(d) != bf(a / 127.0f);
    }
    long inv_bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : inv_bad)
    for (int64_t m = 0; m < (1 << 23); ++m) {
        const float a = fb(0x3F800000u | (uint32_t)m);
        float lo, hi;
        neighbours(a, &lo, &hi);
        const uint32_t want = bf(127.0f / a);
        inv_bad += (bf(inv_fast(a, lo)) != want) + (bf(inv_fast(a, hi)) != want);
    }
    long inv_exp_bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : inv_exp_bad)
    for (int e = -121; e <= 126; ++e)
        for (uint32_t m = 0; m < (1u << 23); m += 509) {
            const float a = ldexpf(fb(0x3F800000u | m), e);
            float lo, hi;
            neighbours(a, &lo, &hi);
            const uint32_t want = bf(127.0f / a);
            inv_exp_bad += (bf(inv_fast(a, lo)) != want) + (bf(inv_fast(a, hi)) != want);
        }
    printf("d_bad %ld\ninv_bad %ld\ninv_exp_bad %ld\n", d_bad, inv_bad, inv_exp_bad);
    return 0;
}
