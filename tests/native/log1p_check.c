/* Exhaustive host check of navi_log1p_nonneg (navi_amd/csrc/log1p_nonneg.h):
 * for every binary32 x in [0, HI] (every STRIDE-th one; STRIDE 1 is every
 * float) the function is within MAX_ULP ulp of the correctly rounded log1p
 * (double log1p, rounded), whichever of RN(1/b) and its two neighbours each of
 * its two navi_recip calls returns (all nine combinations per input): so the
 * bound holds for any reciprocal within one ulp of RN(1/b), such as
 * v_rcp_f32. Also reports how many results differ from the correctly rounded
 * one with correctly rounded reciprocals.
 *
 * Usage: log1p_check [STRIDE] [HI]. Prints the counts and the worst error,
 * exits 1 on a failure. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* navi_recip is called twice per evaluation, for s and then for e / u:
 * g_mode[call] picks -1 (one ulp toward zero), 0 (RN) or +1 (one ulp up). */
static _Thread_local int g_mode[2], g_call;
static inline float navi_recip(float b) {
    const float r = 1.0f / b;
    const int mode = g_mode[g_call++ & 1];
    return mode < 0 ? nextafterf(r, 0.0f) : mode > 0 ? nextafterf(r, INFINITY) : r;
}
#define NAVI_MATH_FN static inline
#include "../../navi_amd/csrc/log1p_nonneg.h"

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t float_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float eval(float x, int ms, int mc) {
    g_mode[0] = ms;
    g_mode[1] = mc;
    g_call = 0;
    return navi_log1p_nonneg(x);
}

#define MAX_ULP 1.0

int main(int argc, char** argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1;
    const float hi = argc > 2 ? (float)atof(argv[2]) : 32.0f;
    int fail = 0;
    const uint32_t last = float_to_bits(hi);
    long n = 0, not_cr = 0, over = 0;
    double worst = 0.0;
    float worst_x = 0.0f;
#pragma omp parallel for schedule(static) reduction(+ : n, not_cr, over)
    for (int64_t i = 0; i <= (int64_t)last; i += stride) {
        const float x = bits_to_float((uint32_t)i);
        const double exact = log1p((double)x);
        const float cr = (float)exact;
        const double ulp = (double)nextafterf(fabsf(cr), INFINITY) - (double)fabsf(cr);
        n++;
        if (float_to_bits(eval(x, 0, 0)) != float_to_bits(cr)) not_cr++;
        double e_max = 0.0;
        for (int ms = -1; ms <= 1; ++ms)
            for (int mc = -1; mc <= 1; ++mc) {
                const double err = fabs((double)eval(x, ms, mc) - exact) / ulp;
                if (err > e_max) e_max = err;
            }
        if (e_max > MAX_ULP) over++;
        if (e_max > worst) {
#pragma omp critical
            if (e_max > worst) {
                worst = e_max;
                worst_x = x;
            }
        }
    }
    /* NaN propagates; zero maps to zero */
    if (!isnan(eval(NAN, 0, 0))) fail = 1;
    if (eval(0.0f, 0, 0) != 0.0f) fail = 1;
    printf("log1p: %ld inputs in [0, %g], %ld not correctly rounded (exact reciprocals), "
           "worst %.4f ulp at x=%a over reciprocal roundings, %ld over %.1f ulp\n",
           n, (double)hi, not_cr, worst, worst_x, over, MAX_ULP);
    if (over) fail = 1;
    return fail;
}
