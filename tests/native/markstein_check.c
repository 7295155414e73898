/* The tracer's exit quotient q = fma(fma(-a*r, b, a), r, a*r), r = RN(1/b),
 * against IEEE division a / b, in the regime the tracer relies on: divisors
 * |b| > 1e-4 (every STRIDE-th float in (1e-4, 16], then sampled up to 2^60),
 * numerators with |a/b| from 1e-7 to 1e4, both signs. Where either result is
 * at least 1e-5 they must be bit-identical; below that (the exit clamps to
 * 1e-5) they must agree on being below it. Prints counts, exits 1 on a miss. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float markstein(float a, float b, float r) {
    float q0 = a * r;
    float e = fmaf(-q0, b, a);
    return fmaf(e, r, q0);
}

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return rng;
}
static double unit(void) { return (double)(next() >> 11) / 9007199254740992.0; }

static long n, bad;
static void check(float a, float b) {
    float r = 1.0f / b, q = a / b, m = markstein(a, b, r);
    n++;
    if (fabsf(q) >= 1e-5f || fabsf(m) >= 1e-5f) {
        if (memcmp(&q, &m, 4)) {
            if (bad < 5) printf("mismatch a=%a b=%a q=%a m=%a\n", a, b, q, m);
            bad++;
        }
    } else if ((q >= 1e-5f) != (m >= 1e-5f)) {
        bad++;
    }
}

int main(int argc, char** argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 64;
    float f = 1e-4f;
    uint32_t lo, hi;
    memcpy(&lo, &f, 4);
    f = 16.0f;
    memcpy(&hi, &f, 4);
    for (uint32_t bb = lo + 1; bb <= hi; bb += stride) {
        float b;
        memcpy(&b, &bb, 4);
        for (int k = 0; k < 4; k++) {
            double qt = pow(10.0, -7.0 + 11.0 * unit());
            float bs = (k & 1) ? -b : b;
            check((float)(qt * (double)bs * ((k & 2) ? -1.0 : 1.0)), bs);
        }
    }
    for (long i = 0; i < 4000000; i++) {
        float b = (float)exp(log(16.0) + (60.0 * log(2.0) - log(16.0)) * unit());
        if (next() & 1) b = -b;
        check((float)(pow(10.0, -7.0 + 11.0 * unit()) * (double)b * ((next() & 1) ? -1.0 : 1.0)), b);
    }
    printf("checked %ld pairs, %ld misses\n", n, bad);
    return bad != 0;
}
