/* log1p_nonneg.h — log(1 + x) in binary32 arithmetic for finite x >= 0 (NaN
 * propagates), within one ulp of the exact value: the log1p of the
 * observation post-pass (torch.log1p of a distance clamped to [0, max],
 * projects/environment/src/navi_environment/backends/sdfdag_backend.py:441
 * of the seismael/navi checkout), at about a third of the instructions of a
 * general-purpose log1pf.
 *
 * Method (the argument reduction of Sun's fdlibm log1p, with Taylor terms):
 *   1 + x = u + e exactly, u = RN(1 + x), e = x - (u - 1);
 *   u = 2^k (1 + f), 1 + f in [sqrt(1/2), sqrt(2)) read off u's bits, f exact
 *   by Sterbenz;
 *   log(1 + f) = 2 atanh(s), s = f / (2 + f), which rearranges to
 *   log(1 + f) = f - f^2/2 + s (f^2/2 + T(s^2)),
 *   T(z) = 2z/3 + 2z^2/5 + 2z^3/7 + 2z^4/9 (|s| < 0.1716, so the dropped
 *   Taylor terms are below 2e-9 of the result);
 *   log(1 + x) = k ln2 + log(1 + f) + e / u, with ln2 split into a 16-bit
 *   head (k ln2_hi exact for k <= 256) and a tail.
 * s enters only the small term s (...). e / u is most of the result for x
 * near 2^-24, so 1/u takes one Newton step after the reciprocal.
 *
 * The includer defines NAVI_MATH_FN (the function's qualifiers) and
 * navi_recip(b), a reciprocal of normal b within one ulp of RN(1 / b).
 * Plain C, so that a host build can check every input against a correctly
 * rounded log1p, for every such reciprocal. */
#ifndef NAVI_LOG1P_NONNEG_H
#define NAVI_LOG1P_NONNEG_H

#include <stdint.h>

NAVI_MATH_FN float navi_log1p_nonneg(float x) {
    const float kLn2Hi = 0x1.62e4p-1f;    /* 0.693145751953125, 16 significant bits */
    const float kLn2Lo = 0x1.7f7d1cp-20f; /* RN(ln2 - kLn2Hi) */
    const uint32_t kSqrtHalf = 0x3f3504f3u; /* bits of RN(sqrt(1/2)) */
    const float u = 1.0f + x;
    /* u - 1 is exact for u >= 1, and so is the rounding error of 1 + x */
    const float e = x - (u - 1.0f);
    /* u = 2^k m, m in [sqrt(1/2), sqrt(2)): offset the bits so that the
     * exponent field carries k */
    uint32_t bu;
    __builtin_memcpy(&bu, &u, 4);
    const int32_t iu = (int32_t)(bu - kSqrtHalf);
    const int32_t k = iu >> 23;
    const uint32_t bm = ((uint32_t)iu & 0x007fffffu) + kSqrtHalf;
    float m;
    __builtin_memcpy(&m, &bm, 4);
    const float f = m - 1.0f;
    const float s = f * navi_recip(2.0f + f);
    const float z = s * s;
    const float t = z * fmaf(z, fmaf(z, fmaf(z, 0x1.c71c72p-3f, 0x1.24924ap-2f), 0x1.99999ap-2f), 0x1.555556p-1f);
    const float hfsq = 0.5f * (f * f);
    const float r = navi_recip(u);
    const float c = e * fmaf(fmaf(-u, r, 1.0f), r, r); /* one Newton step on 1/u */
    const float kf = (float)k;
    return fmaf(kf, kLn2Hi, f - (hfsq - fmaf(s, hfsq + t, fmaf(kf, kLn2Lo, c))));
}

#endif
